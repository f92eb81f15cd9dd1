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

}  // namespace zjai
