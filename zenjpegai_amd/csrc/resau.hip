// ResAU as one kernel (src/model/synthesis.rs:24-74, `ResAu::forward`):
//   t = conv3x3_grouped(relu6(x)), 16 channels per group, no bias;
//   y = x * (1 + conv1x1(t)), no bias (the gate of src/nn/fast/layers.rs:195-201).
// Unfused, t makes a round trip to HBM and the two convolutions are separate launches; for the
// 32- and 64-channel ResAUs of the SOP / BOP luma nets and the HOP chroma net both are small
// (K = 144 and K = C) and launch- and latency-bound on small maps.
//
// One workgroup (4 waves) owns a TR x 16 tile of positions and all C channels:
//   1. relu6(x) over the (TR + 2) x 18 halo -> LDS (storage type; 16-byte units of a pixel XORed
//      with the pixel index so that 16 consecutive pixels' same unit hits different banks);
//   2. wave w computes t for group w % G (G = C / 16) and rows (w / G) * NPW .. : per output,
//      bias-free, the 9 taps in (ky, kx) order, one K chunk of 16 channels (f32:
//      4 x v_mfma_f32_16x16x4_f32; f16 / bf16: one 16x16x32 MFMA whose upper 16 K lanes are the
//      zero padding the unfused kernel also multiplies) -- conv_igemm's instruction sequence for
//      this layer; t is rounded to the storage type into LDS, as the unfused kernel stores it;
//   3. the 1x1 over t for output block w % G on the same rows: K chunks in ascending order, the
//      sequence of conv_igemm / conv1x1_ring for a 1x1 layer; then y = x * (1 + a) as two IEEE
//      operations on the raw x, stored in the storage type.
// The A fragments of both convolutions (9 + C / CK per wave) come straight from global memory
// (the same few KB for every workgroup, L2-resident), so LDS holds only the halo and t and
// several workgroups share a CU. Results equal the two unfused launches bit for bit.

#include "mfma.h"
#include "ops.h"

namespace zjai {

// acc[r] += a . b[r] for N accumulators sharing one A fragment. f32: the four 16x16x4 steps of
// each accumulator in k order, issued k-outermost so that dependent MFMAs are N instructions
// apart (the same per-accumulator sums as Mma16<float>::run).
template <typename T, int N>
__device__ __forceinline__ void mma_rows(f32x4 (&acc)[N], u32x4 a, const u32x4 (&b)[N]) {
    if constexpr (sizeof(T) == 4) {
        const f32x4 af = __builtin_bit_cast(f32x4, a);
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int r = 0; r < N; ++r)
                acc[r] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[k], __builtin_bit_cast(f32x4, b[r])[k], acc[r], 0, 0, 0);
    } else {
#pragma unroll
        for (int r = 0; r < N; ++r) Mma16<T>::run(acc[r], a, b[r]);
    }
}

template <typename T, int C, int TR>
__global__ void __launch_bounds__(256) k_resau(const ResauArgs p) {
    constexpr int VEC = 16 / (int)sizeof(T);  // channels per 16-byte unit
    constexpr int CK = 4 * VEC;               // channels per K chunk (64 bytes)
    constexpr int G = C / 16;                 // groups of 16 channels
    constexpr int UPP = C / VEC;              // 16-byte units per pixel
    constexpr int UG = 16 / VEC;              // units per group
    constexpr int HY = TR + 2, HX = 18, HP = HY * HX;
    constexpr int WPG = 4 / G;                // waves per group
    constexpr int NPW = TR / WPG;             // rows (16-position blocks) per wave
    constexpr int NC2 = C / CK;               // K chunks of the 1x1
    constexpr int HU = HP * UPP, HIT = (HU + 255) / 256;
    static_assert(G == 2 || G == 4, "32 or 64 channels in groups of 16");
    static_assert(TR % WPG == 0 && NPW >= 1, "rows per wave");
    __shared__ u32x4 s_h[HU];
    __shared__ u32x4 s_t[TR * 16 * UPP];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int bid = (int)blockIdx.x;
    const int tx = bid % p.gx, ty = (bid / p.gx) % p.gy, b = bid / (p.gx * p.gy);
    const int y0 = ty * TR, x0 = tx * 16;
    const T* xb = (const T*)p.x.p + (long long)b * p.x.bstride + p.x.c_off;
    const int gi = wave % G;           // group (phase 2) and output block (phase 3)
    const int r0 = (wave / G) * NPW;   // first row of this wave

    // A fragments: grouped 3x3 packing [group][tap][16 out][CK], 1x1 packing [chunk][nblk][16][CK]
    // (16-byte units; lane (col, grp) holds row col, K group grp).
    const u32x4* w1 = (const u32x4*)p.w1 + (long long)gi * 9 * 64;
    const u32x4* w2 = (const u32x4*)p.w2;
    u32x4 a1[9], a2[NC2];
#pragma unroll
    for (int t = 0; t < 9; ++t) a1[t] = w1[(t * 16 + col) * 4 + grp];
#pragma unroll
    for (int c = 0; c < NC2; ++c) a2[c] = w2[((c * p.nblk2 + gi) * 16 + col) * 4 + grp];

    // 1. relu6(x) halo. Every load reads a clamped (in-picture) pixel and off-picture ones take
    // zeros afterwards, so all of a thread's loads are in flight together.
    u32x4 hv[HIT];
#pragma unroll
    for (int i = 0; i < HIT; ++i) {
        const int u = min(tid + i * 256, HU - 1), pix = u / UPP, q = u - pix * UPP;
        const int hy = pix / HX, hx = pix - hy * HX;
        const int cy = min(max(y0 - 1 + hy, 0), p.h - 1), cx = min(max(x0 - 1 + hx, 0), p.w - 1);
        hv[i] = *(const u32x4*)(xb + (long long)cy * p.x.row + (long long)cx * p.x.cs + q * VEC);
    }
#pragma unroll
    for (int i = 0; i < HIT; ++i) {
        const int u = tid + i * 256;
        if (u >= HU) break;
        const int pix = u / UPP, q = u - pix * UPP;
        const int hy = pix / HX, hx = pix - hy * HX;
        const int iy = y0 - 1 + hy, ix = x0 - 1 + hx;
        const bool in = iy >= 0 && iy < p.h && ix >= 0 && ix < p.w;
        s_h[pix * UPP + (q ^ (pix & (UPP - 1)))] = in ? relu6_vec<T>(hv[i]) : u32x4{0u, 0u, 0u, 0u};
    }
    __syncthreads();

    // 2. t for group gi, rows r0 .. r0 + NPW - 1: bias-free, taps (ky, kx) ascending.
    f32x4 acc[NPW];
#pragma unroll
    for (int r = 0; r < NPW; ++r) acc[r] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const int qb = gi * UG + (grp & (UG - 1));  // this lane's unit of the group
#pragma unroll
    for (int t = 0; t < 9; ++t) {
        const int ky = t / 3, kx = t - 3 * (t / 3);
        u32x4 bv[NPW];
#pragma unroll
        for (int r = 0; r < NPW; ++r) {
            const int pix = (r0 + r + ky) * HX + col + kx;
            bv[r] = s_h[pix * UPP + (qb ^ (pix & (UPP - 1)))];
            if (grp >= UG) bv[r] = u32x4{0u, 0u, 0u, 0u};  // 16-bit: K lanes 16..31 are padding
        }
        mma_rows<T, NPW>(acc, a1[t], bv);
    }
    // t (channel gi * 16 + 4 grp + k at position (r0 + r) * 16 + col) rounded to the storage type.
#pragma unroll
    for (int r = 0; r < NPW; ++r) {
        const int pos = (r0 + r) * 16 + col;
        const int ch = gi * 16 + 4 * grp, unit = ch / VEC;
        T* dst = reinterpret_cast<T*>(s_t + pos * UPP + (unit ^ (pos & (UPP - 1)))) + (ch - unit * VEC);
        typedef T t4 __attribute__((ext_vector_type(4)));
        t4 v;
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = (T)acc[r][k];
        *reinterpret_cast<t4*>(dst) = v;
    }
    __syncthreads();

    // 3. a = W2 . t (output block gi), K chunks ascending; y = x * (1 + a).
    f32x4 acc2[NPW];
#pragma unroll
    for (int r = 0; r < NPW; ++r) acc2[r] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < NC2; ++c) {
        u32x4 bv[NPW];
#pragma unroll
        for (int r = 0; r < NPW; ++r) {
            const int pos = (r0 + r) * 16 + col;
            bv[r] = s_t[pos * UPP + ((c * 4 + grp) ^ (pos & (UPP - 1)))];
        }
        mma_rows<T, NPW>(acc2, a2[c], bv);
    }
    T* yb = (T*)p.y.p + (long long)b * p.y.bstride + p.y.c_off;
    const int ch = gi * 16 + 4 * grp;
#pragma unroll
    for (int r = 0; r < NPW; ++r) {
        const int oy = y0 + r0 + r, ox = x0 + col;
        if (oy >= p.h || ox >= p.w) continue;
        const f32x4 xv = load4<T>(xb + (long long)oy * p.x.row + (long long)ox * p.x.cs + ch);
        f32x4 v;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float g = 1.0f + acc2[r][k];
            v[k] = xv[k] * g;
        }
        store4<T>(yb + (long long)oy * p.y.row + (long long)ox * p.y.cs + ch, v);
    }
}

namespace {

template <typename T, int C, int TR>
hipError_t go_resau(ResauArgs p, hipStream_t s) {
    p.gx = (p.w + 15) / 16;
    p.gy = (p.h + TR - 1) / TR;
    const long long total = (long long)p.gx * p.gy * p.N;
    if (total <= 0 || total > (1ll << 30)) return hipErrorInvalidValue;
    hipLaunchKernelGGL((k_resau<T, C, TR>), dim3((unsigned)total), dim3(256), 0, s, p);
    return hipGetLastError();
}

template <typename T>
hipError_t go_resau_t(int C, int tr, const ResauArgs& p, hipStream_t s) {
    if constexpr (sizeof(T) == 4) {
        if (C == 32) return go_resau<T, 32, 8>(p, s);
        if (C == 64) return go_resau<T, 64, 8>(p, s);
    } else {
        if (C == 32) return tr == 8 ? go_resau<T, 32, 8>(p, s) : go_resau<T, 32, 4>(p, s);
        if (C == 64) return tr == 8 ? go_resau<T, 64, 8>(p, s) : go_resau<T, 64, 4>(p, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace

bool resau_fused_supported(int C, int groups) { return (C == 32 || C == 64) && groups * 16 == C; }

int resau_rows(int dtype, int N, int h, int w) {
    // 8-row tiles unless that leaves fewer than 256 workgroups (one per CU). f32 keeps 8 rows:
    // with the fewer accumulators of 4-row tiles the compiler renamed MFMA accumulator chains
    // closer than the ISA guard allows.
    const long long t8 = (long long)((w + 15) / 16) * ((h + 7) / 8) * N;
    return (t8 >= 256 || dtype == DT_F32) ? 8 : 4;
}

hipError_t launch_resau(int dtype, int C, const ResauArgs& p, hipStream_t s) {
    const int vec = dtype == DT_F32 ? 4 : 8;
    if (p.N < 1 || p.N > MAXB || p.h < 1 || p.w < 1 || p.x.cs % vec || p.x.c_off % vec || p.x.row % vec ||
        p.x.bstride % vec || p.y.cs % vec || p.y.c_off % vec || (uintptr_t)p.x.p % 16 || (uintptr_t)p.y.p % 16)
        return hipErrorInvalidValue;
    const int tr = resau_rows(dtype, p.N, p.h, p.w);
    switch (dtype) {
        case DT_F32: return go_resau_t<float>(C, 8, p, s);
        case DT_F16: return go_resau_t<_Float16>(C, tr, p, s);
        case DT_BF16: return go_resau_t<__bf16>(C, tr, p, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace zjai
