// Data movement of the decoder's latent reconstruction (src/decoder/reconstruct.rs:81-234): the
// hyper-decoder's int8 input, the context model's stage merge, the up-shuffled mean of a
// component without a context model, and the region merges of psi and y_hat. The networks
// themselves run on the conv kernels. All of it is HBM-bound data movement at latent resolution.

#include "ops.h"

namespace zjai {

namespace {

inline dim3 blocks_of(long long n) { return dim3((unsigned)((n + 255) / 256)); }

// z_hat int8 planar [C][ZH][ZW], item b's window at (win.x0[b], win.y0[b]) of h x w -> NHWC view,
// exact in every storage type (`Tensor<i8>` -> f32 -> `BTensor::from_planar`,
// src/model/hyper_decoder.rs:66-74).
template <typename T>
__global__ void __launch_bounds__(256) k_i8_planar_to_nhwc(const int8_t* z, int C, int ZH, int ZW, Windows win,
                                                           int N, int h, int w, View dst) {
    const int q = C / 4;
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)N * h * w * q) return;
    const int cq = (int)(i % q);
    long long t = i / q;
    const int x = (int)(t % w);
    t /= w;
    const int y = (int)(t % h), b = (int)(t / h);
    f32x4 v;
#pragma unroll
    for (int k = 0; k < 4; ++k)
        v[k] = (float)z[((long long)(cq * 4 + k) * ZH + win.y0[b] + y) * ZW + win.x0[b] + x];
    store4<T>(at_mut<T>(dst, b, y, x, cq * 4), v);
}

// One context-model stage (ContextModel::decompress_with, src/model/mcm.rs:203-236): the stage's
// mean (NHWC, C channels, hh x hw half-resolution grid) becomes mean + residual where the
// latent sample (2y + py, 2x + px) exists -- one f32 add, in place, so the next stages read it as
// context -- and the same value lands in y_hat (planar [N][C][H][W]). Samples of the padded
// border keep the bare mean and write nothing. Item b's residual window starts at
// (rwin.x0[b], rwin.y0[b]) of a plane with the given row / plane strides.
template <typename T>
__global__ void __launch_bounds__(256) k_mcm_stage(View st, int N, int C, int hh, int hw, const float* res,
                                                   long long res_row, long long res_plane, Windows rwin, int H,
                                                   int W, int py, int px, float* y_hat) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)N * hh * hw * C) return;
    const int c = (int)(i % C);
    long long t = i / C;
    const int x = (int)(t % hw);
    t /= hw;
    const int y = (int)(t % hh), b = (int)(t / hh);
    const int sy = 2 * y + py, sx = 2 * x + px;
    if (sy >= H || sx >= W) return;
    T* p = at_mut<T>(st, b, y, x, c);
    const float v = to_f32(*p) + res[(long long)c * res_plane + (long long)(rwin.y0[b] + sy) * res_row + rwin.x0[b] + sx];
    *p = from_f32<T>(v);
    y_hat[(((long long)b * C + c) * H + sy) * W + sx] = v;
}

// A component without a context model (src/decoder/reconstruct.rs:191-202): the psi quarters
// up-shuffled to latent resolution (`upshuffle_psi_par`, src/model/mcm.rs:742-764: stage
// (y % 2, x % 2) -> quarter {0, 2, 3, 1}) plus the residual, one f32 add per sample.
template <typename T>
__global__ void __launch_bounds__(256) k_upshuffle_psi(View psi, int N, int C, const float* res, long long res_row,
                                                       long long res_plane, Windows rwin, int H, int W,
                                                       float* y_hat) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)N * C * H * W) return;
    const int x = (int)(i % W);
    long long t = i / W;
    const int y = (int)(t % H);
    t /= H;
    const int c = (int)(t % C), b = (int)(t / C);
    const int quarter = (0x1320 >> (4 * ((y & 1) * 2 + (x & 1)))) & 0xf;  // {0, 2, 3, 1}
    const float m = to_f32(*at<T>(psi, b, y >> 1, x >> 1, quarter * C + c));
    y_hat[i] = m + res[(long long)c * res_plane + (long long)(rwin.y0[b] + y) * res_row + rwin.x0[b] + x];
}

// `assign_par` (src/decoder/reconstruct.rs:38-62) from an NHWC tile: dst[c][dy0 + y][dx0 + x] =
// src[oy + y][ox + x][c] over the clamped h x w rectangle; x fastest for the planar writes.
template <typename T>
__global__ void __launch_bounds__(256) k_assign_from_nhwc(View src, int C, int oy, int ox, int h, int w,
                                                          float* dst, int DH, int DW, int dy0, int dx0) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)C * h * w) return;
    const int x = (int)(i % w);
    const long long t = i / w;
    const int y = (int)(t % h), c = (int)(t / h);
    dst[((long long)c * DH + dy0 + y) * DW + dx0 + x] = to_f32(*at<T>(src, 0, oy + y, ox + x, c));
}

// `assign_par` between planar f32 planes: dst[c][dy0 + y][dx0 + x] = src[c][oy + y][ox + x].
__global__ void __launch_bounds__(256) k_assign_planar(const float* src, int C, int SH, int SW, int oy, int ox,
                                                       int h, int w, float* dst, int DH, int DW, int dy0,
                                                       int dx0) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)C * h * w) return;
    const int x = (int)(i % w);
    const long long t = i / w;
    const int y = (int)(t % h), c = (int)(t / h);
    dst[((long long)c * DH + dy0 + y) * DW + dx0 + x] = src[((long long)c * SH + oy + y) * SW + ox + x];
}

}  // namespace

#define ZJAI_LATENT_DISPATCH(dtype, KERNEL, ...)                                              \
    switch (dtype) {                                                                         \
        case DT_F32: KERNEL<float> __VA_ARGS__; break;                                       \
        case DT_F16: KERNEL<_Float16> __VA_ARGS__; break;                                    \
        case DT_BF16: KERNEL<__bf16> __VA_ARGS__; break;                                     \
        default: return hipErrorInvalidValue;                                                \
    }

hipError_t launch_i8_planar_to_nhwc(const int8_t* z, int C, int ZH, int ZW, const Windows& win, int N, int h, int w,
                                    View dst, int dtype, hipStream_t s) {
    if (C % 4 || N < 1 || N > MAXB) return hipErrorInvalidValue;
    for (int b = 0; b < N; ++b)
        if (win.y0[b] < 0 || win.x0[b] < 0 || win.y0[b] + h > ZH || win.x0[b] + w > ZW) return hipErrorInvalidValue;
    const long long n = (long long)N * h * w * (C / 4);
    if (n <= 0) return hipSuccess;
    ZJAI_LATENT_DISPATCH(dtype, k_i8_planar_to_nhwc, <<<blocks_of(n), 256, 0, s>>>(z, C, ZH, ZW, win, N, h, w, dst))
    return hipGetLastError();
}

hipError_t launch_mcm_stage(View st, int dtype, int N, int C, int hh, int hw, const float* res, long long res_row,
                            long long res_plane, const Windows& rwin, int H, int W, int py, int px, float* y_hat,
                            hipStream_t s) {
    if (N < 1 || N > MAXB || 2 * hh < H || 2 * hw < W || py < 0 || py > 1 || px < 0 || px > 1)
        return hipErrorInvalidValue;
    const long long n = (long long)N * hh * hw * C;
    if (n <= 0) return hipSuccess;
    ZJAI_LATENT_DISPATCH(dtype, k_mcm_stage, <<<blocks_of(n), 256, 0, s>>>(st, N, C, hh, hw, res, res_row, res_plane,
                                                                           rwin, H, W, py, px, y_hat))
    return hipGetLastError();
}

hipError_t launch_upshuffle_psi(View psi, int dtype, int N, int C, int ph, int pw, const float* res, long long res_row,
                                long long res_plane, const Windows& rwin, int H, int W, float* y_hat, hipStream_t s) {
    if (N < 1 || N > MAXB || 2 * ph < H || 2 * pw < W) return hipErrorInvalidValue;
    const long long n = (long long)N * C * H * W;
    if (n <= 0) return hipSuccess;
    ZJAI_LATENT_DISPATCH(dtype, k_upshuffle_psi,
                         <<<blocks_of(n), 256, 0, s>>>(psi, N, C, res, res_row, res_plane, rwin, H, W, y_hat))
    return hipGetLastError();
}

hipError_t launch_assign_from_nhwc(View src, int dtype, int C, int SH, int SW, int oy, int ox, int h, int w,
                                   float* dst, int DH, int DW, int dy0, int dx0, hipStream_t s) {
    if (h <= 0 || w <= 0 || C <= 0) return hipSuccess;
    if (oy < 0 || ox < 0 || oy + h > SH || ox + w > SW || dy0 < 0 || dx0 < 0 || dy0 + h > DH || dx0 + w > DW)
        return hipErrorInvalidValue;
    const long long n = (long long)C * h * w;
    ZJAI_LATENT_DISPATCH(dtype, k_assign_from_nhwc,
                         <<<blocks_of(n), 256, 0, s>>>(src, C, oy, ox, h, w, dst, DH, DW, dy0, dx0))
    return hipGetLastError();
}

hipError_t launch_assign_planar(const float* src, int C, int SH, int SW, int oy, int ox, int h, int w, float* dst,
                                int DH, int DW, int dy0, int dx0, hipStream_t s) {
    if (h <= 0 || w <= 0 || C <= 0) return hipSuccess;
    if (oy < 0 || ox < 0 || oy + h > SH || ox + w > SW || dy0 < 0 || dx0 < 0 || dy0 + h > DH || dx0 + w > DW)
        return hipErrorInvalidValue;
    const long long n = (long long)C * h * w;
    k_assign_planar<<<blocks_of(n), 256, 0, s>>>(src, C, SH, SW, oy, ox, h, w, dst, DH, DW, dy0, dx0);
    return hipGetLastError();
}

}  // namespace zjai
