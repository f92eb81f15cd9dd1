// Data movement of the analysis transforms (src/model/analysis.rs, encoder side): the input
// normalisation with the first replicate padding, the replicate padding before each stride-2
// convolution, and the optional per-channel feature clipping. The convolutions, ResAU, TAM and
// CAB blocks run on the synthesis kernels. HBM-bound, read and write once.

#include "ops.h"

namespace zjai {

namespace {

inline dim3 blocks_of(long long n) { return dim3((unsigned)((n + 255) / 256)); }

// `normalize` ((x - 127.5) / 128, src/model/analysis.rs:35-39) of planar f32 [C][H][W] in
// [0, 255], written as NHWC of Cp >= C channels (zero beyond C) and OH x OW >= H x W samples,
// where rows / columns past the picture replicate the last one (`padding_layer`,
// src/model/analysis.rs:43-81). x fastest, so the planar reads coalesce.
template <typename T>
__global__ void __launch_bounds__(256) k_normalize_pad(const float* x, int C, int H, int W, int Cp, int OH,
                                                       int OW, View dst) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)OH * OW * (Cp / 4)) return;
    const int xo = (int)(i % OW);
    const long long t = i / OW;
    const int yo = (int)(t % OH), cq = (int)(t / OH);
    const int sy = min(yo, H - 1), sx = min(xo, W - 1);
    f32x4 v;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int c = cq * 4 + k;
        v[k] = c < C ? (x[((long long)c * H + sy) * W + sx] - 127.5f) / 128.0f : 0.0f;
    }
    store4<T>(at_mut<T>(dst, 0, yo, xo, cq * 4), v);
}

// `replicate_pad` (src/model/analysis.rs:48-70): NHWC H x W -> OH x OW, new rows / columns copy
// the last ones.
template <typename T>
__global__ void __launch_bounds__(256) k_replicate_pad(View src, int N, int C, int H, int W, View dst, int OH,
                                                       int OW) {
    const int q = C / 4;
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)N * OH * OW * q) return;
    const int cq = (int)(i % q);
    long long t = i / q;
    const int xo = (int)(t % OW);
    t /= OW;
    const int yo = (int)(t % OH), b = (int)(t / OH);
    store4<T>(at_mut<T>(dst, b, yo, xo, cq * 4), load4<T>(at<T>(src, b, min(yo, H - 1), min(xo, W - 1), cq * 4)));
}

// `clip_channels` (src/model/load.rs:103-119): channel c < n clamped to [lo[c], hi[c]] in place
// (`f32::clamp`: NaN stays NaN).
template <typename T>
__global__ void __launch_bounds__(256) k_clip_channels(View x, int N, int H, int W, int n, const float* lo,
                                                       const float* hi) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)N * H * W * n) return;
    const int c = (int)(i % n);
    long long t = i / n;
    const int xo = (int)(t % W);
    t /= W;
    const int yo = (int)(t % H), b = (int)(t / H);
    T* p = at_mut<T>(x, b, yo, xo, c);
    float v = to_f32(*p);
    if (v < lo[c]) v = lo[c];
    if (v > hi[c]) v = hi[c];
    *p = from_f32<T>(v);
}

}  // namespace

#define ZJAI_ANALYSIS_DISPATCH(dtype, KERNEL, ...)                                            \
    switch (dtype) {                                                                         \
        case DT_F32: KERNEL<float> __VA_ARGS__; break;                                       \
        case DT_F16: KERNEL<_Float16> __VA_ARGS__; break;                                    \
        case DT_BF16: KERNEL<__bf16> __VA_ARGS__; break;                                     \
        default: return hipErrorInvalidValue;                                                \
    }

hipError_t launch_normalize_pad(const float* x, int C, int H, int W, int Cp, int OH, int OW, View dst, int dtype,
                                hipStream_t s) {
    if (C <= 0 || H <= 0 || W <= 0 || Cp < C || Cp % 4 || OH < H || OW < W) return hipErrorInvalidValue;
    const long long n = (long long)OH * OW * (Cp / 4);
    ZJAI_ANALYSIS_DISPATCH(dtype, k_normalize_pad, <<<blocks_of(n), 256, 0, s>>>(x, C, H, W, Cp, OH, OW, dst))
    return hipGetLastError();
}

hipError_t launch_replicate_pad(View src, int dtype, int N, int C, int H, int W, View dst, int OH, int OW,
                                hipStream_t s) {
    if (N < 1 || C <= 0 || C % 4 || H <= 0 || W <= 0 || OH < H || OW < W) return hipErrorInvalidValue;
    const long long n = (long long)N * OH * OW * (C / 4);
    ZJAI_ANALYSIS_DISPATCH(dtype, k_replicate_pad, <<<blocks_of(n), 256, 0, s>>>(src, N, C, H, W, dst, OH, OW))
    return hipGetLastError();
}

hipError_t launch_clip_channels(View x, int dtype, int N, int C, int H, int W, int n, const float* lo,
                                const float* hi, hipStream_t s) {
    if (n < 0 || n > C || N < 1) return hipErrorInvalidValue;
    const long long total = (long long)N * H * W * n;
    if (total <= 0) return hipSuccess;
    ZJAI_ANALYSIS_DISPATCH(dtype, k_clip_channels, <<<blocks_of(total), 256, 0, s>>>(x, N, H, W, n, lo, hi))
    return hipGetLastError();
}

}  // namespace zjai
