// Device-side helpers shared by the synthesis kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace zjai {

// Storage types of activations and packed weights.
enum DType : int { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2 };

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

// A batched NHWC activation view: element (b, y, x, c) lives at
// p[b * bstride + y * row + x * cs + c_off + c]. Batch items are synthesis tiles of one shape.
struct View {
    void* p;
    long long row;
    long long bstride;
    int cs;
    int c_off;
};

template <typename T>
__device__ __forceinline__ const T* at(const View& v, int b, int y, int x, int c) {
    return (const T*)v.p + (long long)b * v.bstride + (long long)y * v.row + (long long)x * v.cs + v.c_off + c;
}
template <typename T>
__device__ __forceinline__ T* at_mut(const View& v, int b, int y, int x, int c) {
    return (T*)v.p + (long long)b * v.bstride + (long long)y * v.row + (long long)x * v.cs + v.c_off + c;
}

// Largest number of tiles one launch batches.
constexpr int MAXB = 8;

template <typename T> struct Elem;
template <> struct Elem<float> { static constexpr int dt = DT_F32; };
template <> struct Elem<_Float16> { static constexpr int dt = DT_F16; };
template <> struct Elem<__bf16> { static constexpr int dt = DT_BF16; };

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(_Float16 v) { return (float)v; }
__device__ __forceinline__ float to_f32(__bf16 v) { return (float)v; }

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ _Float16 from_f32<_Float16>(float v) { return (_Float16)v; }
template <> __device__ __forceinline__ __bf16 from_f32<__bf16>(float v) { return (__bf16)v; }

// Four consecutive channels, loaded / stored as one vector access.
template <typename T> __device__ __forceinline__ f32x4 load4(const T* p);
template <> __device__ __forceinline__ f32x4 load4<float>(const float* p) {
    return *reinterpret_cast<const f32x4*>(p);
}
template <> __device__ __forceinline__ f32x4 load4<_Float16>(const _Float16* p) {
    f16x4 h = *reinterpret_cast<const f16x4*>(p);
    return f32x4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
}
template <> __device__ __forceinline__ f32x4 load4<__bf16>(const __bf16* p) {
    bf16x4 h = *reinterpret_cast<const bf16x4*>(p);
    return f32x4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
}
template <typename T> __device__ __forceinline__ void store4(T* p, f32x4 v);
template <> __device__ __forceinline__ void store4<float>(float* p, f32x4 v) {
    *reinterpret_cast<f32x4*>(p) = v;
}
template <> __device__ __forceinline__ void store4<_Float16>(_Float16* p, f32x4 v) {
    *reinterpret_cast<f16x4*>(p) = f16x4{(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
}
template <> __device__ __forceinline__ void store4<__bf16>(__bf16* p, f32x4 v) {
    *reinterpret_cast<bf16x4*>(p) = bf16x4{(__bf16)v[0], (__bf16)v[1], (__bf16)v[2], (__bf16)v[3]};
}

// Cephes expf as straight IEEE operations, as the reference's `nn::fast::math::exp`
// (src/nn/fast/math.rs:28-62). All HIP sources build with -ffp-contract=off, so none of these
// multiply/add pairs fuse.
__device__ __forceinline__ float cephes_exp(float x) {
    x = x < -87.0f ? -87.0f : x;
    x = x > 88.0f ? 88.0f : x;
    float t = x * 1.44269504088896340736f;
    t = t + 0.5f;
    const float n = floorf(t);
    float r = x - n * 0.693359375f;
    r = r - n * -2.12194440e-4f;
    float p = 1.9875691500e-4f;
    p = p * r; p = p + 1.3981999507e-3f;
    p = p * r; p = p + 8.3334519073e-3f;
    p = p * r; p = p + 4.1665795894e-2f;
    p = p * r; p = p + 1.6666665459e-1f;
    p = p * r; p = p + 5.0000001201e-1f;
    float y = p * (r * r);
    y = y + r;
    y = y + 1.0f;
    // y * 2^n. After the clamps n is an integer in [-126, 127] (x = -87 gives n = -126), so 2^n
    // is a normal float and the product is exact scaling with one rounding: v_ldexp_f32 gives the
    // same bits as multiplying by the constructed power of two. The clamps are comparisons, so a
    // NaN x reaches here with n NaN; converting NaN to int is undefined, so it takes 0 instead
    // (y is NaN then, and so is the result).
    const int ni = (n != n) ? 0 : (int)n;
    return ldexpf(y, ni);
}

// ELU(a) = a > 0 ? a : exp(a) - 1 for the 16-bit storage paths' transformer gate, with exp from
// the hardware's 2^x (v_exp_f32 on a * log2 e; for a <= 0 the error of exp(a) - 1 stays within
// ~1e-7 absolute, far below the f16 / bf16 rounding of the gate's result) instead of the Cephes
// polynomial the f32 path keeps for parity with the reference (src/nn/fast/math.rs:74-80). One transcendental and a multiply against ~25 vector
// instructions: the feed-forward's gate phase is bound by its vector ALUs.
__device__ __forceinline__ float elu_fast16(float a) {
    const float e = __builtin_amdgcn_exp2f(a * 1.44269504088896340736f) - 1.0f;
    return a > 0.0f ? a : e;
}

__device__ __forceinline__ float sigmoidf_ref(float x) {
    const float e = cephes_exp(-x);
    return 1.0f / (1.0f + e);
}

}  // namespace zjai
