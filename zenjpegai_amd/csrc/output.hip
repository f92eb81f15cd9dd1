// The decoder's output stage on the device (src/decoder/output.rs): chroma resampling to the
// source format and the BT.709 -> RGB conversion with its quantisation, over the float planes a
// picture run leaves in HBM.
//
// Resampling restates PyTorch's CPU kernels the way the reference pins them, operation for
// operation (its tests/nn_vectors.rs checks them bit for bit against PyTorch):
//   * bicubic, align_corners (`resize_bicubic`, output.rs:100-147): scale = (in-1)/(out-1),
//     real = scale * dst, base = floor(real), t = real - base, taps clamp(base-1+k); A = -0.75
//     weights in the fused forms of :64-79; four horizontal dot4 (x1*c1, then fma with x0, x2,
//     x3; :85-90), then the vertical dot4 over them;
//   * bilinear, align_corners (`nn::resize_bilinear`, src/nn/resample.rs:22-69): i0 = (int)real,
//     i1 = i0 + (i0 < in-1), l1 = real - i0; equal sizes map straight through; corner weights
//     pre-multiplied and accumulated fma(p0, a, p1*b), fma(p2, c, .), fma(p3, d, .).
// One thread per output sample; the picture kernel samples U and V bicubically at its own pixel
// (the same per-sample arithmetic as the resampler), so the full-size chroma planes never exist.
// All of it is HBM-bound: per RGB pixel 4 bytes of luma, the chroma taps (cache hits) and 6
// bytes of uint16 RGB (+ 12 bytes of float RGB planes when asked for).

#include "ops.h"

namespace zjai {

namespace {

__device__ __forceinline__ float cubic1(float x) {
    const float A = -0.75f;
    const float p = fmaf(A + 2.0f, x, -(A + 3.0f));
    return fmaf(p * x, x, 1.0f);
}

__device__ __forceinline__ float cubic2(float x) {
    const float A = -0.75f;
    float p = fmaf(A, x, -5.0f * A);
    p = fmaf(p, x, 8.0f * A);
    return fmaf(p, x, -4.0f * A);
}

__device__ __forceinline__ float dot4(const float (&x)[4], const float (&c)[4]) {
    float acc = x[1] * c[1];
    acc = fmaf(x[0], c[0], acc);
    acc = fmaf(x[2], c[2], acc);
    return fmaf(x[3], c[3], acc);
}

struct Cubic {
    int idx[4];
    float wt[4];
};

// Source taps and weights of output coordinate dst (align_corners); scale is
// (in - 1) / (out - 1) in f32, computed once on the host.
__device__ __forceinline__ Cubic cubic_taps(int dst, int in_len, float scale) {
    Cubic c;
    const float real = scale * (float)dst;
    const float basef = floorf(real);
    const float t = real - basef;
    const int base = (int)basef;
#pragma unroll
    for (int k = 0; k < 4; ++k) c.idx[k] = min(max(base - 1 + k, 0), in_len - 1);
    const float u = 1.0f - t;
    c.wt[0] = cubic2(t + 1.0f);
    c.wt[1] = cubic1(t);
    c.wt[2] = cubic1(u);
    c.wt[3] = cubic2(u + 1.0f);
    return c;
}

__device__ __forceinline__ float bicubic_at(const float* plane, int w, const Cubic& cy, const Cubic& cx) {
    float rows[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float* row = plane + (long long)cy.idx[k] * w;
        const float v[4] = {row[cx.idx[0]], row[cx.idx[1]], row[cx.idx[2]], row[cx.idx[3]]};
        rows[k] = dot4(v, cx.wt);
    }
    return dot4(rows, cy.wt);
}

__global__ void __launch_bounds__(256) k_resize_bicubic(const float* src, int c, int h, int w,
                                                        float* dst, int oh, int ow, float sy,
                                                        float sx) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long n = (long long)c * oh * ow;
    if (i >= n) return;
    const int x = (int)(i % ow), y = (int)((i / ow) % oh), ch = (int)(i / ((long long)oh * ow));
    const Cubic cy = cubic_taps(y, h, sy), cx = cubic_taps(x, w, sx);
    dst[i] = bicubic_at(src + (long long)ch * h * w, w, cy, cx);
}

struct Linear {
    int i0, i1;
    float l0, l1;
};

__device__ __forceinline__ Linear linear_taps(int dst, int in_len, int out_len, float scale) {
    Linear t;
    if (in_len == out_len) {
        t.i0 = t.i1 = dst;
        t.l0 = 1.0f;
        t.l1 = 0.0f;
        return t;
    }
    const float real = scale * (float)dst;
    const int a = (int)real;
    t.i0 = a;
    t.i1 = a + (a < in_len - 1 ? 1 : 0);
    t.l1 = real - (float)a;
    t.l0 = 1.0f - t.l1;
    return t;
}

__global__ void __launch_bounds__(256) k_resize_bilinear(const float* src, int c, int h, int w,
                                                         float* dst, int oh, int ow, float sy,
                                                         float sx) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long n = (long long)c * oh * ow;
    if (i >= n) return;
    const int x = (int)(i % ow), y = (int)((i / ow) % oh), ch = (int)(i / ((long long)oh * ow));
    const Linear ty = linear_taps(y, h, oh, sy), tx = linear_taps(x, w, ow, sx);
    const float p0 = ty.l0 * tx.l0, p1 = ty.l0 * tx.l1, p2 = ty.l1 * tx.l0, p3 = ty.l1 * tx.l1;
    const float* sp = src + (long long)ch * h * w;
    const float* r0 = sp + (long long)ty.i0 * w;
    const float* r1 = sp + (long long)ty.i1 * w;
    float acc = fmaf(p0, r0[tx.i0], p1 * r0[tx.i1]);
    acc = fmaf(p2, r1[tx.i0], acc);
    dst[i] = fmaf(p3, r1[tx.i1], acc);
}

// convert_range(x, a, b) = ((x - 0) / a) * b + 0 (output.rs:36-40), each step an IEEE op.
__device__ __forceinline__ float convert_range(float x, float in_max, float out_max) {
    float v = x - 0.0f;
    v = v / in_max;
    v = v * out_max;
    return v + 0.0f;
}

__device__ __forceinline__ float clamp255(float v) { return v < 0.0f ? 0.0f : (v > 255.0f ? 255.0f : v); }

// BT.709 (output.rs:27-33): the constants combined in f64 and narrowed to f32 (:225-228).
constexpr double KR = 0.2126, KG = 0.7152, KB = 0.0722, KBY = 1.8556, KRY = 1.5748;

// One picture pixel: luma (H x W) and chroma planes (ch x cw, bicubic to H x W unless equal)
// -> clipped RGB (to_rgb_planes_owned_par, output.rs:232-257) -> uint16 interleaved
// (quantize_par, :407-437) and, when rgbf is set, the float planes [3][H][W].
__global__ void __launch_bounds__(256) k_picture_rgb(const float* y, int H, int W, const float* u,
                                                     const float* v, int ch, int cw, float sy,
                                                     float sx, float qmax, uint16_t* rgb,
                                                     float* rgbf) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)H * W) return;
    const int px = (int)(i % W), py = (int)(i / W);
    float us, vs;
    if (ch == H && cw == W) {
        us = u[i];
        vs = v[i];
    } else {
        const Cubic cy = cubic_taps(py, ch, sy), cx = cubic_taps(px, cw, sx);
        us = bicubic_at(u, cw, cy, cx);
        vs = bicubic_at(v, cw, cy, cx);
    }
    const float kry = (float)KRY, kby = (float)KBY;
    const float gu = (float)(KB * KBY / KG), gv = (float)(KR * KRY / KG);
    const float yy = convert_range(y[i], 255.0f, 1.0f);
    const float uu = convert_range(us, 255.0f, 1.0f) - 0.5f;
    const float vv = convert_range(vs, 255.0f, 1.0f) - 0.5f;
    const float rv = yy + kry * vv;
    float gvv = yy - gu * uu;
    gvv = gvv - gv * vv;
    const float bv = yy + kby * uu;
    const float c3[3] = {clamp255(convert_range(rv, 1.0f, 255.0f)), clamp255(convert_range(gvv, 1.0f, 255.0f)),
                         clamp255(convert_range(bv, 1.0f, 255.0f))};
    uint16_t q[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        float s = rintf(convert_range(c3[k], 255.0f, qmax));
        s = s < 0.0f ? 0.0f : (s > qmax ? qmax : s);
        q[k] = (uint16_t)s;
        if (rgbf) rgbf[(long long)k * H * W + i] = c3[k];
    }
    uint16_t* d = rgb + i * 3;
    d[0] = q[0];
    d[1] = q[1];
    d[2] = q[2];
}

inline float align_scale(int in_len, int out_len) {
    return out_len > 1 ? (float)(in_len - 1) / (float)(out_len - 1) : 0.0f;
}

inline unsigned blocks_for(long long n) { return (unsigned)((n + 255) / 256); }

}  // namespace

hipError_t launch_resize(int mode, const float* src, int c, int h, int w, float* dst, int oh, int ow,
                         hipStream_t s) {
    const long long n = (long long)c * oh * ow;
    if (n <= 0) return hipSuccess;
    if (n / 256 >= 0x7fffffffLL) return hipErrorInvalidValue;
    const float sy = align_scale(h, oh), sx = align_scale(w, ow);
    if (mode == RESIZE_BICUBIC)
        k_resize_bicubic<<<blocks_for(n), 256, 0, s>>>(src, c, h, w, dst, oh, ow, sy, sx);
    else if (mode == RESIZE_BILINEAR)
        k_resize_bilinear<<<blocks_for(n), 256, 0, s>>>(src, c, h, w, dst, oh, ow, sy, sx);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_picture_rgb(const float* y, int H, int W, const float* u, const float* v, int ch,
                              int cw, int bit_depth, uint16_t* rgb, float* rgbf, hipStream_t s) {
    const long long n = (long long)H * W;
    if (n <= 0) return hipSuccess;
    if (n / 256 >= 0x7fffffffLL || ch <= 0 || cw <= 0) return hipErrorInvalidValue;
    const float qmax = (float)((1u << bit_depth) - 1);
    k_picture_rgb<<<blocks_for(n), 256, 0, s>>>(y, H, W, u, v, ch, cw, align_scale(ch, H),
                                                align_scale(cw, W), qmax, rgb, rgbf);
    return hipGetLastError();
}

}  // namespace zjai
