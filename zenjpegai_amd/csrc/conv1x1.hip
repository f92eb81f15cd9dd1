// 1x1 convolutions (stride 1, no padding, one group) as a GEMM: output channels x positions,
// K = input channels, in every storage type.
//
// A workgroup of WC x WP waves computes NB * 16 output channels (NB = WC * CF 16-channel
// blocks) for MP = WP * PF * 16 consecutive positions of one batch item (positions are the
// row-major pixel index of the output map, so narrow maps waste no lanes). The K loop streams
// 64 bytes of input channels per position per chunk (16 f32 or 32 f16 / bf16 channels) with
// direct global -> LDS loads (global_load_lds_dwordx4: lane i's 16 bytes land at the wave's LDS
// base + 16 i) through a ring of NS chunk slots, one barrier per chunk, NS - 2 chunks in flight
// behind the one being consumed. A position's 64 bytes are read by 4 consecutive lanes as one
// contiguous run; its 4 16-byte slots are XOR-swizzled by the position index so that the
// fragment reads are free of bank conflicts (as are the weight rows'). The weight blocks are
// the implicit-GEMM packing ([chunk][16-channel block][16][64 bytes]), one contiguous NB-block
// run per chunk.
//
// Numerics are those of the implicit-GEMM kernels for a 1x1 layer, so the two agree bit for
// bit: the bias first, then chunk by chunk in ascending order; f32 as four
// v_mfma_f32_16x16x4_f32 per chunk (k = 0..3, the K group of lane group g holding channels
// 4g + k), f16 / bf16 as one v_mfma_f32_16x16x32 per chunk (lane group g holding channels
// 8g..8g+7). The epilogue is the shared one (epilogue.h) through an LDS transpose.
//
// On the config-5 layer shapes (202 500 positions) this runs within 10-20 % of the vendor BLAS
// on the same plain GEMM (f32 128 -> 1024: 663 vs 608 us; bf16 128 -> 384: 74 vs 83 us) with
// the residual epilogue fused; persistent workgroups with a ring across tiles and a variant
// that loads the fragments straight into registers (no LDS, no barriers) were both slower.

#include "conv.h"
#include "epilogue.h"
#include "mfma.h"

namespace zjai {

__device__ u32x4 g_zero_units1x1[4];  // 64 zero bytes: the source of positions past the map

// s_waitcnt with vmcnt(n) (expcnt and lgkmcnt not waited for): gfx9 keeps vmcnt's low four
// bits in [3:0] and its high two bits in [15:14].
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

template <typename T, int WC, int WP, int CF, int PF, int NS, int TP, int WPE>
__global__ void __launch_bounds__(WC * WP * 64) __attribute__((amdgpu_waves_per_eu(WPE)))
conv1x1_ring(const ConvParams p) {
    constexpr int NT = WC * WP * 64;
    constexpr int NB = WC * CF;
    constexpr int MP = WP * PF * 16;
    constexpr int VEC = 16 / (int)sizeof(T);
    constexpr int B_U = MP * 4;   // one chunk of positions: [MP][4 swizzled 16-byte slots]
    constexpr int A_U = NB * 64;  // one chunk of weights: [NB][64 units]
    constexpr int STG_U = B_U + A_U;
    constexpr int OUT_LD = NB * 16 + 4;
    constexpr int PP = MP / TP;  // positions per epilogue pass
    constexpr int OUT_U = (PP * OUT_LD + 3) / 4;
    constexpr int LDS_U = (NS * STG_U) > OUT_U ? (NS * STG_U) : OUT_U;
    constexpr int BN = B_U / NT, AN = A_U / NT;
    constexpr int L = BN + AN;  // loads per thread and chunk
    static_assert(B_U % NT == 0 && A_U % NT == 0 && NS >= 2 && (NS - 2) * L < 64, "tile");
    static_assert(PP % 16 == 0 && MP % TP == 0, "epilogue passes cover whole 16-position blocks");
    __shared__ u32x4 s_lds[LDS_U];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wc = wave % WC, wp = wave / WC;
    const int col = lane & 15, grp = lane >> 4;

    // XCD-aware order (conv.hip's scheme): logical order (batch, position tile, channel tile)
    // with the channel tiles of one position tile consecutive on one XCD (shared input in L2).
    const int P = p.OH * p.OW;
    const int ptiles = (P + MP - 1) / MP;
    const int nct = p.ntiles;
    const int total = p.N * ptiles * nct;
    const int bid = (int)blockIdx.x, xj = bid & 7, xk = bid >> 3;
    const int q8 = total >> 3, r8 = total & 7;
    const int lid = xj < r8 ? xj * (q8 + 1) + xk : r8 * (q8 + 1) + (xj - r8) * q8 + xk;
    int rest = lid / nct;
    const int ct = lid - rest * nct;
    const int pt = rest % ptiles, bi = rest / ptiles;
    const int pos0 = pt * MP, nb0 = ct * NB;

    f32x4 acc[CF][PF];
#pragma unroll
    for (int cf = 0; cf < CF; ++cf) {
        const int oc = (nb0 + wc * CF + cf) * 16 + grp * 4;
        f32x4 b;
#pragma unroll
        for (int i = 0; i < 4; ++i) b[i] = p.bias ? p.bias[oc + i] : 0.0f;
#pragma unroll
        for (int pf = 0; pf < PF; ++pf) acc[cf][pf] = b;
    }

    const T* xg = (const T*)p.x.p + (long long)bi * p.x.bstride + p.x.c_off;
    const u32x4* wg = (const u32x4*)((const T*)p.w + (long long)bi * p.w_bstride) + (long long)nb0 * 64;
    const long long wchunk = (long long)p.nblk_g * 64;  // units between consecutive chunks

    // Element offset of each of this thread's position units (u = tid + i * NT), -1 past the
    // map: unit u = position * 4 + slot holds the position's 16-byte unit slot ^ swz(position),
    // swz(position) = 2 (bit 2 of the position). A fragment read (ds_read_b128, lane (col, grp))
    // runs in four passes of 16 lanes (lane l in pass (l / 32, parity of bits 2..4 of l)) over
    // 64 banks; with this swizzle each pass's 16 units sit on distinct bank quads. The weight
    // rows take the same swizzle (unit q of row r at q ^ swz(r)).
    long long boff[BN];
#pragma unroll
    for (int i = 0; i < BN; ++i) {
        const int u = tid + i * NT, pos = u >> 2, slot = u & 3;
        const int q = slot ^ ((pos & 4) >> 1);
        const int pg = pos0 + pos;
        if (pg < P) {
            const int oy = pg / p.OW, ox = pg - oy * p.OW;
            boff[i] = (long long)oy * p.x.row + (long long)ox * p.x.cs + q * VEC;
        } else {
            boff[i] = -1;
        }
    }

    // Direct LDS loads of chunk c into ring slot c % NS (L instructions per thread).
    auto issue = [&](int c) __attribute__((always_inline)) {
        u32x4* dst = s_lds + (c % NS) * STG_U;
        const long long c0 = (long long)c * 4 * VEC;
#pragma unroll
        for (int i = 0; i < BN; ++i) {
            const void* src = boff[i] >= 0 ? (const void*)(xg + boff[i] + c0) : (const void*)g_zero_units1x1;
            lds_dma16(src, dst + wave * 64 + i * NT);
        }
#pragma unroll
        for (int i = 0; i < AN; ++i) {
            const int u = wave * 64 + i * NT;
            const int U = u + lane;  // LDS unit U holds weight unit U ^ swz(row U / 4)
            lds_dma16(wg + c * wchunk + (U ^ ((U >> 3) & 2)), dst + B_U + u);
        }
    };

    int bpos[PF];
#pragma unroll
    for (int pf = 0; pf < PF; ++pf) bpos[pf] = (wp * PF + pf) * 16 + col;

    // Ring of NS chunks: chunk c + NS - 1 is issued once every wave has passed chunk c's barrier
    // (so all are done with chunk c - 1, whose slot it takes); NS - 2 chunks stay in flight
    // behind the one being waited for (loads complete in issue order).
    const int nch = p.nchunks;
#pragma unroll
    for (int c = 0; c < NS - 1; ++c)
        if (c < nch) issue(c);
    for (int c = 0; c < nch; ++c) {
        if (c + NS - 2 < nch) wait_vmcnt<(NS - 2) * L>();
        else wait_vmcnt<0>();
        __syncthreads();
        if (c + NS - 1 < nch) issue(c + NS - 1);
        const u32x4* sb = s_lds + (c % NS) * STG_U;
        const u32x4* sa = sb + B_U;
        u32x4 av[CF], bv[PF];
#pragma unroll
        for (int cf = 0; cf < CF; ++cf) av[cf] = sa[(wc * CF + cf) * 64 + col * 4 + (grp ^ ((col & 4) >> 1))];
#pragma unroll
        for (int pf = 0; pf < PF; ++pf) {
            const int pos = bpos[pf];
            bv[pf] = sb[pos * 4 + (grp ^ ((pos & 4) >> 1))];
        }
        if constexpr (sizeof(T) == 4) {
            // k outermost: the four dependent MFMAs of an accumulator are CF x PF apart.
#pragma unroll
            for (int k = 0; k < 4; ++k)
#pragma unroll
                for (int cf = 0; cf < CF; ++cf)
#pragma unroll
                    for (int pf = 0; pf < PF; ++pf)
                        acc[cf][pf] = __builtin_amdgcn_mfma_f32_16x16x4f32(__builtin_bit_cast(f32x4, av[cf])[k],
                                                                           __builtin_bit_cast(f32x4, bv[pf])[k],
                                                                           acc[cf][pf], 0, 0, 0);
        } else {
#pragma unroll
            for (int cf = 0; cf < CF; ++cf)
#pragma unroll
                for (int pf = 0; pf < PF; ++pf) Mma16<T>::run(acc[cf][pf], av[cf], bv[pf]);
        }
    }

    // Epilogue: transpose through LDS so that consecutive threads store consecutive channels of
    // one position, TP passes of PP positions (a 16-position fragment lies in one pass).
    float* so = reinterpret_cast<float*>(s_lds);
    const int oc0 = nb0 * 16;
    const bool simple = epilogue_simple(p), ps2 = epilogue_ps2(p);
#pragma unroll
    for (int pass = 0; pass < TP; ++pass) {
        __syncthreads();
#pragma unroll
        for (int pf = 0; pf < PF; ++pf) {
            if (((wp * PF + pf) * 16) / PP != pass) continue;  // uniform per wave
#pragma unroll
            for (int cf = 0; cf < CF; ++cf)
                *reinterpret_cast<f32x4*>(so + (bpos[pf] - pass * PP) * OUT_LD + (wc * CF + cf) * 16 + grp * 4) =
                    acc[cf][pf];
        }
        __syncthreads();
        if (simple) {
            constexpr int QP8 = NB * 2;
#pragma unroll 4
            for (int u = tid; u < PP * QP8; u += NT) {
                const int pos = u / QP8, c8 = u - pos * QP8;
                const int pg = pos0 + pass * PP + pos;
                const f32x4 v0 = *reinterpret_cast<const f32x4*>(so + pos * OUT_LD + c8 * 8);
                const f32x4 v1 = *reinterpret_cast<const f32x4*>(so + pos * OUT_LD + c8 * 8 + 4);
                if (pg < P) {
                    const int oy = pg / p.OW, ox = pg - oy * p.OW;
                    epilogue_store8<T>(p, bi, oy, ox, oc0 + c8 * 8, v0, v1);
                }
            }
        } else if (ps2) {
            // Unit u: position, sub-position s, output-channel quad cq (conv channels
            // 16 cq + 4 j + s, j = 0..3, of this tile).
#pragma unroll 2
            for (int u = tid; u < PP * 4 * NB; u += NT) {
                const int pos = u / (4 * NB), r = u - pos * (4 * NB), s = r / NB, cq = r - s * NB;
                const int pg = pos0 + pass * PP + pos;
                if (pg >= P) continue;
                const int oy = pg / p.OW, ox = pg - oy * p.OW;
                const float* sv = so + pos * OUT_LD + 16 * cq + s;
                epilogue_store_ps2<T>(p, bi, oy, ox, s, oc0 / 4 + 4 * cq, f32x4{sv[0], sv[4], sv[8], sv[12]});
            }
        } else {
            constexpr int QP = NB * 4;
            for (int u = tid; u < PP * QP; u += NT) {
                const int pos = u / QP, cq = u - pos * QP;
                const int pg = pos0 + pass * PP + pos;
                if (pg >= P) continue;
                const int oy = pg / p.OW, ox = pg - oy * p.OW;
                const f32x4 v = *reinterpret_cast<const f32x4*>(so + pos * OUT_LD + cq * 4);
                epilogue_store<T>(p, bi, oy, ox, oc0 + cq * 4, 4, v);
            }
        }
    }
}

template <typename T, int WC, int WP, int CF, int PF, int NS, int TP, int WPE>
static hipError_t go_1x1(const ConvParams& p0, hipStream_t s) {
    constexpr int NB = WC * CF, MP = WP * PF * 16;
    ConvParams p = p0;
    p.ntiles = p.cout_g / (NB * 16);
    const long long ptiles = ((long long)p.OH * p.OW + MP - 1) / MP;
    const long long total = ptiles * p.N * p.ntiles;
    if (p.nblk_g % NB || p.cout_g % (NB * 16) || total <= 0 || total > (1ll << 30)) return hipErrorInvalidValue;
    hipLaunchKernelGGL((conv1x1_ring<T, WC, WP, CF, PF, NS, TP, WPE>), dim3((unsigned)total), dim3(WC * WP * 64), 0, s,
                       p);
    return hipGetLastError();
}

// A view whose channel groups of 4 start on 4-element boundaries (the epilogue's vector stores
// and residual loads).
static bool aligned4(const View& v) { return !(v.cs % 4) && !(v.c_off % 4) && !(v.row % 4) && !(v.bstride % 4); }

bool conv1x1_ring_ok(const ConvParams& p, int dtype) {
    const int vec = dtype == DT_F32 ? 4 : 8;
    return p.groups == 1 && p.N >= 1 && p.N <= MAXB && !p.relu6_in && p.H == p.OH && p.W == p.OW &&
           p.pad_t == 0 && p.pad_l == 0 && p.cin_g % (4 * vec) == 0 && p.nchunks * 4 * vec == p.cin_g &&
           p.cout_g % 64 == 0 && p.nblk_g % 4 == 0 && p.x.cs % vec == 0 && p.x.c_off % vec == 0 &&
           p.x.row % vec == 0 && p.x.bstride % vec == 0 && aligned4(p.y) && (!p.r1.p || aligned4(p.r1)) &&
           (!p.r2.p || aligned4(p.r2));
}

int conv1x1_ring_nb(const ConvParams& p) { return (p.cout_g % 128 == 0 && p.nblk_g % 8 == 0) ? 8 : 4; }

template <typename T>
static hipError_t go_1x1_t(const ConvParams& p, hipStream_t s) {
    // Co-resident workgroups cover each other's prologue and epilogue. f32: a ring of 3 chunks and
    // two epilogue passes (48 KB of LDS, <= 168 registers: 3 workgroups per CU); 16-bit, whose
    // layers are HBM-bound: a ring of 2 and four passes (32 KB, <= 128 registers: 4 per CU).
    // Against a ring of 4 and one pass (2 per CU) on 202 500 positions: f32 128 -> 1024 664 ->
    // 617 us, 128 -> 384 268 -> 239 us; bf16 128 -> 1024 223 -> 172 us, 512 -> 128 85 -> 74 us,
    // 128 -> 384 76 -> 55 us (4 per CU: f32 no better, bf16 a further 7-10 %).
    if constexpr (sizeof(T) == 4) {
        if (conv1x1_ring_nb(p) == 8) return go_1x1<T, 2, 2, 4, 4, 3, 2, 3>(p, s);  // 128 ch x 128 positions
        return go_1x1<T, 1, 4, 4, 2, 3, 2, 3>(p, s);                                 // 64 ch x 128 positions
    } else {
        if (conv1x1_ring_nb(p) == 8) return go_1x1<T, 2, 2, 4, 4, 2, 4, 4>(p, s);
        return go_1x1<T, 1, 4, 4, 2, 2, 4, 4>(p, s);
    }
}

hipError_t launch_conv1x1_ring(int dtype, const ConvParams& p, hipStream_t s) {
    if (!conv1x1_ring_ok(p, dtype)) return hipErrorInvalidValue;
    switch (dtype) {
        case DT_F32: return go_1x1_t<float>(p, s);
        case DT_F16: return go_1x1_t<_Float16>(p, s);
        case DT_BF16: return go_1x1_t<__bf16>(p, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace zjai
