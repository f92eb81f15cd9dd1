// Bandwidth-bound kernels: layout changes, elementwise ops, depthwise 3x3, layer norm and the
// reductions of channel attention. Element order and rounding follow the reference's
// `nn::fast::{layers, depthwise, math}` (each op a separate IEEE operation, FMA only where the
// reference's contract has one).

#include "ops.h"

namespace zjai {

template <typename T>
__device__ __forceinline__ const T* at(const View& v, int y, int x, int c) {
    return (const T*)v.p + (long long)y * v.row + (long long)x * v.cs + v.c_off + c;
}
template <typename T>
__device__ __forceinline__ T* at_mut(const View& v, int y, int x, int c) {
    return (T*)v.p + (long long)y * v.row + (long long)x * v.cs + v.c_off + c;
}

// ------------------------------------------------------------------------------ layout moves
template <typename T>
__global__ void k_planar_to_nhwc(const float* src, int C, int LH, int LW, int x0, int y0, int h,
                                 int w, View dst) {
    const int q = C / 4;
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)h * w * q) return;
    const int cq = (int)(i % q);
    const long long pos = i / q;
    const int x = (int)(pos % w), y = (int)(pos / w);
    f32x4 v;
#pragma unroll
    for (int k = 0; k < 4; ++k)
        v[k] = src[((long long)(cq * 4 + k) * LH + (y0 + y)) * LW + (x0 + x)];
    store4<T>(at_mut<T>(dst, y, x, cq * 4), v);
}

template <typename T>
__global__ void k_nhwc_to_planar(View src, int C, int h, int w, float* dst) {
    const int q = (C + 3) / 4;
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)h * w * q) return;
    const int x = (int)(i % w);
    const long long r = i / w;
    const int y = (int)(r % h), cq = (int)(r / h);
    for (int k = 0; k < 4; ++k) {
        const int c = cq * 4 + k;
        if (c < C) dst[((long long)c * h + y) * w + x] = to_f32(*at<T>(src, y, x, c));
    }
}

template <typename T>
__global__ void k_copy(View src, View dst, int C, int h, int w) {
    const int q = C / 4;
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)h * w * q) return;
    const int cq = (int)(i % q);
    const long long pos = i / q;
    const int x = (int)(pos % w), y = (int)(pos / w);
    store4<T>(at_mut<T>(dst, y, x, cq * 4), load4<T>(at<T>(src, y, x, cq * 4)));
}

template <typename T>
__global__ void k_pixel_shuffle(View src, View dst, int C, int h, int w, int r) {
    const int q = C / 4, oh = h * r, ow = w * r;
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)oh * ow * q) return;
    const int cq = (int)(i % q);
    const long long pos = i / q;
    const int X = (int)(pos % ow), Y = (int)(pos / ow);
    const int y = Y / r, dy = Y - y * r, x = X / r, dx = X - x * r;
    f32x4 v;
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = to_f32(*at<T>(src, y, x, (cq * 4 + k) * r * r + dy * r + dx));
    store4<T>(at_mut<T>(dst, Y, X, cq * 4), v);
}

// ---------------------------------------------------------------------------------- eltwise
template <typename T>
__global__ void k_eltwise(int op, View xv, View sv, int C, int h, int w) {
    const int q = C / 4;
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)h * w * q) return;
    const int cq = (int)(i % q);
    const long long pos = i / q;
    const int x = (int)(pos % w), y = (int)(pos / w);
    T* px = at_mut<T>(xv, y, x, cq * 4);
    f32x4 v = load4<T>(px);
    f32x4 s = {0, 0, 0, 0};
    if (op >= EL_ADD) s = load4<T>(at<T>(sv, y, x, cq * 4));
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        float e = v[k];
        switch (op) {
            case EL_RELU: e = fmaxf(e, 0.0f); break;
            case EL_RELU6: e = e < 0.0f ? 0.0f : e; e = e > 6.0f ? 6.0f : e; break;
            case EL_LEAKY: e = e < 0.0f ? e * 0.01f : e; break;
            case EL_SIGMOID: e = sigmoidf_ref(e); break;
            case EL_ADD: e = e + s[k]; break;
            case EL_GATE: { const float g = 1.0f + s[k]; e = e * g; } break;
            case EL_MUL: e = e * s[k]; break;
            case EL_ELU_GATE: {
                const float ex = cephes_exp(e) - 1.0f;
                const float elu = e > 0.0f ? e : ex;
                e = elu * s[k];
            } break;
        }
        v[k] = e;
    }
    store4<T>(px, v);
}

// ------------------------------------------------------------------------- depthwise 3x3
// Per output element: acc = bias; for ky, kx ascending: acc = fma(w, x, acc), padding taps
// included (src/nn/fast/depthwise.rs:40-73). Weights are stored transposed, [9][C].
template <typename T>
__global__ void k_depthwise3x3(View src, View dst, int C, int h, int w, const float* wt,
                               const float* bias, int elu_half) {
    const int cout = elu_half > 0 ? elu_half : C;
    const int q = cout / 4;
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)h * w * q) return;
    const int cq = (int)(i % q);
    const long long pos = i / q;
    const int x = (int)(pos % w), y = (int)(pos / w);
    const int npass = elu_half > 0 ? 2 : 1;
    f32x4 res[2];
    for (int pass = 0; pass < npass; ++pass) {
        const int c0 = cq * 4 + pass * elu_half;
        f32x4 acc;
#pragma unroll
        for (int k = 0; k < 4; ++k) acc[k] = bias ? bias[c0 + k] : 0.0f;
#pragma unroll
        for (int ky = 0; ky < 3; ++ky) {
            const int yy = y + ky - 1;
#pragma unroll
            for (int kx = 0; kx < 3; ++kx) {
                const int xx = x + kx - 1;
                f32x4 xv = {0.0f, 0.0f, 0.0f, 0.0f};
                if (yy >= 0 && yy < h && xx >= 0 && xx < w) xv = load4<T>(at<T>(src, yy, xx, c0));
                const f32x4 wv = *(const f32x4*)(wt + (ky * 3 + kx) * C + c0);
#pragma unroll
                for (int k = 0; k < 4; ++k) acc[k] = fmaf(wv[k], xv[k], acc[k]);
            }
        }
        res[pass] = acc;
    }
    f32x4 out = res[0];
    if (elu_half > 0) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float a = res[0][k];
            const float e = cephes_exp(a) - 1.0f;
            const float elu = a > 0.0f ? a : e;
            out[k] = elu * res[1][k];
        }
    }
    store4<T>(at_mut<T>(dst, y, x, cq * 4), out);
}

// ------------------------------------------------------------------------------ layer norm
// `layer_norm_channels` (src/nn/fast/math.rs:423-448): f64 sums over channels in order,
// (x - mean) / sqrt(var + 1e-5) * w + b with f32 operations.
template <typename T>
__global__ void k_layer_norm(View src, View dst, int C, int h, int w, const float* wt,
                             const float* bs) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)h * w) return;
    const int x = (int)(i % w), y = (int)(i / w);
    const T* p = at<T>(src, y, x, 0);
    double mean = 0.0;
    for (int c = 0; c < C; c += 4) {
        const f32x4 v = load4<T>(p + c);
        mean += (double)v[0]; mean += (double)v[1]; mean += (double)v[2]; mean += (double)v[3];
    }
    mean /= (double)C;
    double var = 0.0;
    for (int c = 0; c < C; c += 4) {
        const f32x4 v = load4<T>(p + c);
#pragma unroll
        for (int k = 0; k < 4; ++k) { const double d = (double)v[k] - mean; var = var + d * d; }
    }
    const float m32 = (float)mean;
    const float den = sqrtf((float)(var / (double)C) + 1e-5f);
    T* o = at_mut<T>(dst, y, x, 0);
    for (int c = 0; c < C; c += 4) {
        const f32x4 v = load4<T>(p + c);
        f32x4 r;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float e = v[k] - m32;
            e = e / den;
            e = e * wt[c + k];
            r[k] = e + bs[c + k];
        }
        store4<T>(o + c, r);
    }
}

// ------------------------------------------------------------------------ channel attention
// Gram partial sums: per chunk of ATT_POS positions, entries per head are q_i.k_j (c*c),
// |q_i|^2 (c) and |k_j|^2 (c). f32 products accumulated in f32 per chunk, stored as f64.
constexpr int ATT_POS = 256, ATT_SUB = 32, ATT_MAXE = 20;

int attention_gram_chunks(int h, int w) { return (h * w + ATT_POS - 1) / ATT_POS; }

template <typename T>
__global__ void __launch_bounds__(256) k_attention_gram(View qkv, int dim, int heads, int h, int w,
                                                        double* partial) {
    extern __shared__ float s_qk[];  // [ATT_SUB][2*dim]
    const int c = dim / heads, E = c * c + 2 * c, total = heads * E;
    const int n = h * w, tid = threadIdx.x;
    float acc[ATT_MAXE];
    int ea[ATT_MAXE], eb[ATT_MAXE];
#pragma unroll
    for (int k = 0; k < ATT_MAXE; ++k) {
        acc[k] = 0.0f;
        const int e = tid + k * 256;
        ea[k] = eb[k] = -1;
        if (e < total) {
            const int hd = e / E, r = e - hd * E;
            if (r < c * c) { ea[k] = hd * c + r / c; eb[k] = dim + hd * c + r % c; }
            else if (r < c * c + c) { ea[k] = eb[k] = hd * c + (r - c * c); }
            else { ea[k] = eb[k] = dim + hd * c + (r - c * c - c); }
        }
    }
    const int base = blockIdx.x * ATT_POS;
    for (int sub = 0; sub < ATT_POS; sub += ATT_SUB) {
        __syncthreads();
        for (int u = tid; u < ATT_SUB * (2 * dim / 4); u += 256) {
            const int pl = u / (2 * dim / 4), cq = u - pl * (2 * dim / 4);
            const int p = base + sub + pl;
            f32x4 v = {0, 0, 0, 0};
            if (p < n) v = load4<T>(at<T>(qkv, p / w, p % w, cq * 4));
            *(f32x4*)&s_qk[pl * 2 * dim + cq * 4] = v;
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < ATT_MAXE; ++k) {
            if (ea[k] < 0) continue;
            float a = acc[k];
            for (int pl = 0; pl < ATT_SUB; ++pl) a = fmaf(s_qk[pl * 2 * dim + ea[k]], s_qk[pl * 2 * dim + eb[k]], a);
            acc[k] = a;
        }
    }
#pragma unroll
    for (int k = 0; k < ATT_MAXE; ++k) {
        const int e = tid + k * 256;
        if (e < total) partial[(long long)blockIdx.x * total + e] = (double)acc[k];
    }
}

// Reduce partials, normalise (F.normalize eps 1e-12), scale by temperature, softmax with the
// Cephes exp and an f64 sum (src/nn/fast/math.rs:560-577), then fold the projection.
__global__ void __launch_bounds__(256) k_attention_softmax_fold(const double* partial, int nchunk,
                                                                int dim, int heads,
                                                                const float* temperature,
                                                                const float* proj, float* attn,
                                                                float* wfold) {
    extern __shared__ double s_red[];  // [heads * E]
    const int c = dim / heads, E = c * c + 2 * c, total = heads * E, tid = threadIdx.x;
    for (int e = tid; e < total; e += 256) {
        double s = 0.0;
        for (int k = 0; k < nchunk; ++k) s += partial[(long long)k * total + e];
        s_red[e] = s;
    }
    __syncthreads();
    // One thread per attention row (dim rows).
    float* sm = (float*)(s_red + total);  // [dim][c] scratch rows
    for (int row = tid; row < dim; row += 256) {
        const int hd = row / c, i = row - hd * c;
        const double* S = s_red + hd * E;
        float nq = (float)sqrt(S[c * c + i]);
        nq = nq > 1e-12f ? nq : 1e-12f;
        float mx = -INFINITY;
        for (int j = 0; j < c; ++j) {
            float nk = (float)sqrt(S[c * c + c + j]);
            nk = nk > 1e-12f ? nk : 1e-12f;
            const float a = (float)(S[i * c + j] / ((double)nq * (double)nk)) * temperature[hd];
            sm[row * c + j] = a;
            mx = fmaxf(mx, a);
        }
        double sum = 0.0;
        for (int j = 0; j < c; ++j) {
            const float e = cephes_exp(sm[row * c + j] - mx);
            sm[row * c + j] = e;
            sum += (double)e;
        }
        const float s32 = (float)sum;
        for (int j = 0; j < c; ++j) {
            const float a = sm[row * c + j] / s32;
            sm[row * c + j] = a;
            attn[row * c + j] = a;
        }
    }
    __syncthreads();
    // wfold[o][hd*c + j] = sum_i proj[o][hd*c + i] * attn[hd*c + i][j]  (f64 accumulate)
    for (int e = tid; e < dim * dim; e += 256) {
        const int o = e / dim, col = e - o * dim, hd = col / c, j = col - hd * c;
        double s = 0.0;
        for (int i = 0; i < c; ++i) s += (double)proj[o * dim + hd * c + i] * (double)sm[(hd * c + i) * c + j];
        wfold[e] = (float)s;
    }
}

// ------------------------------------------------------------------------------- launchers
static inline dim3 grid_for(long long n) { return dim3((unsigned)((n + 255) / 256)); }

#define ZJAI_DISPATCH(dtype, KERNEL, ...)                                                     \
    switch (dtype) {                                                                         \
        case DT_F32: KERNEL<float> __VA_ARGS__; break;                                       \
        case DT_F16: KERNEL<_Float16> __VA_ARGS__; break;                                    \
        case DT_BF16: KERNEL<__bf16> __VA_ARGS__; break;                                     \
        default: return hipErrorInvalidValue;                                                \
    }

hipError_t launch_planar_to_nhwc(const float* src, int C, int LH, int LW, int x0, int y0, int h,
                                 int w, View dst, int dtype, hipStream_t s) {
    const long long n = (long long)h * w * (C / 4);
    if (n == 0) return hipSuccess;
    ZJAI_DISPATCH(dtype, k_planar_to_nhwc, <<<grid_for(n), 256, 0, s>>>(src, C, LH, LW, x0, y0, h, w, dst))
    return hipGetLastError();
}

hipError_t launch_nhwc_to_planar(View src, int dtype, int C, int h, int w, float* dst,
                                 hipStream_t s) {
    const long long n = (long long)h * w * ((C + 3) / 4);
    if (n == 0) return hipSuccess;
    ZJAI_DISPATCH(dtype, k_nhwc_to_planar, <<<grid_for(n), 256, 0, s>>>(src, C, h, w, dst))
    return hipGetLastError();
}

hipError_t launch_eltwise(int op, View x, View src, int dtype, int C, int h, int w, hipStream_t s) {
    const long long n = (long long)h * w * (C / 4);
    if (n == 0) return hipSuccess;
    ZJAI_DISPATCH(dtype, k_eltwise, <<<grid_for(n), 256, 0, s>>>(op, x, src, C, h, w))
    return hipGetLastError();
}

hipError_t launch_copy(View src, View dst, int dtype, int C, int h, int w, hipStream_t s) {
    const long long n = (long long)h * w * (C / 4);
    if (n == 0) return hipSuccess;
    ZJAI_DISPATCH(dtype, k_copy, <<<grid_for(n), 256, 0, s>>>(src, dst, C, h, w))
    return hipGetLastError();
}

hipError_t launch_pixel_shuffle(View src, View dst, int dtype, int C_out, int h, int w, int r,
                                hipStream_t s) {
    const long long n = (long long)h * r * w * r * (C_out / 4);
    if (n == 0) return hipSuccess;
    ZJAI_DISPATCH(dtype, k_pixel_shuffle, <<<grid_for(n), 256, 0, s>>>(src, dst, C_out, h, w, r))
    return hipGetLastError();
}

hipError_t launch_depthwise3x3(View src, View dst, int dtype, int C, int h, int w,
                               const float* weight, const float* bias, int elu_half,
                               hipStream_t s) {
    const int cout = elu_half > 0 ? elu_half : C;
    const long long n = (long long)h * w * (cout / 4);
    if (n == 0) return hipSuccess;
    ZJAI_DISPATCH(dtype, k_depthwise3x3, <<<grid_for(n), 256, 0, s>>>(src, dst, C, h, w, weight, bias, elu_half))
    return hipGetLastError();
}

hipError_t launch_layer_norm(View src, View dst, int dtype, int C, int h, int w,
                             const float* weight, const float* bias, hipStream_t s) {
    const long long n = (long long)h * w;
    if (n == 0) return hipSuccess;
    ZJAI_DISPATCH(dtype, k_layer_norm, <<<grid_for(n), 256, 0, s>>>(src, dst, C, h, w, weight, bias))
    return hipGetLastError();
}

hipError_t launch_attention_gram(View qkv, int dtype, int dim, int heads, int h, int w,
                                 double* partial, hipStream_t s) {
    const int c = dim / heads;
    if (heads * (c * c + 2 * c) > 256 * ATT_MAXE) return hipErrorInvalidValue;
    const int nchunk = attention_gram_chunks(h, w);
    if (nchunk == 0) return hipSuccess;
    const size_t lds = sizeof(float) * ATT_SUB * 2 * dim;
    ZJAI_DISPATCH(dtype, k_attention_gram, <<<dim3(nchunk), 256, lds, s>>>(qkv, dim, heads, h, w, partial))
    return hipGetLastError();
}

hipError_t launch_attention_softmax_fold(const double* partial, int nchunk, int dim, int heads,
                                         const float* temperature, const float* proj,
                                         float* attn, float* wfold, hipStream_t s) {
    const int c = dim / heads, total = heads * (c * c + 2 * c);
    const size_t lds = sizeof(double) * total + sizeof(float) * dim * c;
    k_attention_softmax_fold<<<1, 256, lds, s>>>(partial, nchunk, dim, heads, temperature, proj,
                                                 attn, wfold);
    return hipGetLastError();
}

}  // namespace zjai
