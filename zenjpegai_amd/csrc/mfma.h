// Matrix-core fragments shared by the HIP kernels (gfx950 / CDNA4, wave64).
#pragma once

#include "device.h"

namespace zjai {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// 16x16 tile, 32 channels of K per instruction for the 16-bit types (four 16x16x4 steps for
// f32). Lane (i, g) = (lane % 16, lane / 16) supplies row / column i and K group g (8 channels
// of a 16-bit type, 4 of f32); accumulator register r holds row 4 * g + r of column i.
template <typename T> struct Mma16;
template <> struct Mma16<float> {
    static __device__ __forceinline__ void run(f32x4& acc, u32x4 a, u32x4 b) {
        const f32x4 av = __builtin_bit_cast(f32x4, a), bv = __builtin_bit_cast(f32x4, b);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[0], bv[0], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[1], bv[1], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[2], bv[2], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[3], bv[3], acc, 0, 0, 0);
    }
};
template <> struct Mma16<_Float16> {
    static __device__ __forceinline__ void run(f32x4& acc, u32x4 a, u32x4 b) {
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                     __builtin_bit_cast(f16x8, b), acc, 0, 0, 0);
    }
};
template <> struct Mma16<__bf16> {
    static __device__ __forceinline__ void run(f32x4& acc, u32x4 a, u32x4 b) {
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                      __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
    }
};

// 32x32 tile, 16 channels of K per instruction (16-bit types only): v_mfma_f32_32x32x16 runs
// at twice the rate of the 16x16x32 form on gfx950 (measured 2.36 vs 1.33 PF/s on register
// operands). Lane (j, h) = (lane % 32, lane / 32) supplies row / column j and channels
// 8h..8h+7 of the 16-channel step; accumulator register r holds row 8 * (r / 4) + 4 * h + r % 4
// of column j.
template <typename T> struct Mma32;
template <> struct Mma32<_Float16> {
    static __device__ __forceinline__ void run(f32x16& acc, u32x4 a, u32x4 b) {
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                     __builtin_bit_cast(f16x8, b), acc, 0, 0, 0);
    }
};
template <> struct Mma32<__bf16> {
    static __device__ __forceinline__ void run(f32x16& acc, u32x4 a, u32x4 b) {
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                      __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
    }
};

// Direct global -> LDS load of 16 bytes per lane (global_load_lds_dwordx4): lane i's bytes land
// at wave_dst + 16 i (wave_dst is the wave's base; its value in lane 0 is used). Written as
// inline assembly because the compiler counts its own form of this load as LDS work still in
// flight and then waits for every outstanding LDS read (lgkmcnt(0)) wherever a kernel first uses
// the result of any one of them, which serialises the fragment reads a tap loop issues ahead of
// its MFMAs; hidden from it, each use waits only for the reads it needs. The compiler does not
// count these loads in its own vmcnt waits either: the caller waits for them (s_waitcnt
// vmcnt(0), then the barrier that publishes the LDS data) before any wave reads the bytes.
// (The s_nop is the wait state a write of M0 needs before an LDS DMA instruction reads it.)
__device__ __forceinline__ void lds_dma16(const void* src, void* wave_dst) {
    const unsigned m0 = __builtin_amdgcn_readfirstlane(
        (unsigned)(size_t)(__attribute__((address_space(3))) void*)wave_dst);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(src), "s"(m0)
                 : "memory", "m0");
}

// clamp(v, 0, 6) on a 16-byte vector of the storage type (ResAU's relu6 on load).
template <typename T> __device__ __forceinline__ u32x4 relu6_vec(u32x4 v);
template <> __device__ __forceinline__ u32x4 relu6_vec<float>(u32x4 v) {
    f32x4 f = __builtin_bit_cast(f32x4, v);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float e = f[i];
        e = e < 0.0f ? 0.0f : e;
        e = e > 6.0f ? 6.0f : e;
        f[i] = e;
    }
    return __builtin_bit_cast(u32x4, f);
}
template <> __device__ __forceinline__ u32x4 relu6_vec<_Float16>(u32x4 v) {
    f16x8 h = __builtin_bit_cast(f16x8, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        _Float16 e = h[i];
        e = e < (_Float16)0.0f ? (_Float16)0.0f : e;
        e = e > (_Float16)6.0f ? (_Float16)6.0f : e;
        h[i] = e;
    }
    return __builtin_bit_cast(u32x4, h);
}
template <> __device__ __forceinline__ u32x4 relu6_vec<__bf16>(u32x4 v) {
    bf16x8 h = __builtin_bit_cast(bf16x8, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float e = (float)h[i];
        e = e < 0.0f ? 0.0f : e;
        e = e > 6.0f ? 6.0f : e;
        h[i] = (__bf16)e;
    }
    return __builtin_bit_cast(u32x4, h);
}

}  // namespace zjai
