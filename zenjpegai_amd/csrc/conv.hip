// Implicit-GEMM convolution on CDNA4 matrix cores (gfx950).
//
// One workgroup computes TY = WP*PF output rows x 16 output columns x NB = WC*CF blocks of 16
// output channels. GEMM roles: M = output channels (the weights are the A operand), N = output
// positions (the input halo is the B operand), K = input channels x taps.
//
// Per input-channel chunk (64 bytes of channels per pixel: 16 f32 or 32 f16/bf16) the workgroup
// stages the input halo [HY][HX][64 B] and the packed weights [NB][taps][16][64 B] in LDS, then
// every wave runs, per tap, one 16-byte LDS read per operand fragment and CF x PF MFMAs:
//   f32:      4 x v_mfma_f32_16x16x4_f32 (lane group g holds channels 4g..4g+3)
//   f16/bf16: 1 x v_mfma_f32_16x16x32_{f16,bf16} (lane group g holds channels 8g..8g+7)
// A and B fragments use the same lane-group -> channel map, so each MFMA sums matching channels.
// Accumulators start at the bias; the epilogue applies activation, residual op, pixel shuffle,
// denormalisation and quantisation, and stores NHWC activations or planar picture samples.
//
// Transposed stride-2 convolutions run as four output phases (blockIdx.z & 3): each phase is a
// stride-1 gather over the input with at most 2x2 taps whose input offsets lie in {-1, 0, 1},
// so the halo is the 3x3 one and only the tap table differs.

#include "conv.h"
#include "epilogue.h"
#include "mfma.h"

#include <type_traits>

namespace zjai {

// The 16x16 fragment of mfma.h (Mma16): 4 x 16x16x4 f32 steps or one 16x16x32 16-bit step.
template <typename T> using Mma = Mma16<T>;

// Staged operands keep 4 16-byte units (one K group each) per row: a halo slot or a weight row,
// unit q of row r at q ^ qswz(r). A fragment read (ds_read_b128) takes 16 consecutive rows x 4
// K groups, lane (row, group) = (lane % 16, lane / 16). gfx950 serves such a read in four
// passes of 16 lanes, lane l in pass (l / 32, parity of bits 2..4 of l), 16 bytes per bank
// quad, 64 banks: unswizzled, each pass holds two lanes per bank quad (2-way conflicts);
// flipping bit 1 of the unit index in rows with bit 2 set spreads every pass over all banks,
// for any first row, and keeps the 8-lane passes of the register-staged 16-byte stores
// conflict-free too (measured with rocprofv3's SQ_LDS_BANK_CONFLICT on lane-pattern probes).
__device__ __forceinline__ int qswz(int r) { return (r & 4) >> 1; }

// SG: input-channel chunks staged per barrier. 1x1 layers do little matrix work per chunk, so
// they stage several (SG = 4: the whole K of a 128-channel f16 layer) with every global load of
// the stage issued before its LDS stores -- more bytes in flight per workgroup, fewer barriers.
__device__ u32x4 g_zero_igemm[1];  // 16 zero bytes: the source of padding units

template <typename T, int KH, int KW, int S, bool TR, int WC, int WP, int CF, int PF, int SG>
__global__ void __launch_bounds__(WC * WP * 64)
conv_igemm(const ConvParams p) {
    constexpr int NT = WC * WP * 64;
    constexpr int TY = WP * PF;
    constexpr int HY = (TY - 1) * S + KH;
    constexpr int HX = 15 * S + KW;
    constexpr int NTAP = TR ? 4 : KH * KW;
    constexpr int NB = WC * CF;
    constexpr int VEC = 16 / (int)sizeof(T);
    constexpr int CK = 4 * VEC;
    constexpr int HALO_U = HY * HX * 4;
    constexpr int W_U = NB * NTAP * 64;
    // The output tile [TY * 16 positions][NB * 16 + 4 channels] (f32) reuses the same LDS after
    // the K loop (the +4 pads rows against bank conflicts).
    constexpr int OUT_LD = NB * 16 + 4;
    constexpr int OUT_U = (TY * 16 * OUT_LD + 3) / 4;
    constexpr int STG_U = HALO_U + W_U;
    constexpr int LDS_U = (SG * STG_U) > OUT_U ? (SG * STG_U) : OUT_U;
    constexpr int HN = (HALO_U + NT - 1) / NT, WN = (W_U + NT - 1) / NT;
    __shared__ u32x4 s_lds[LDS_U];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wc = wave % WC, wp = wave / WC;
    const int col = lane & 15, grp = lane >> 4;

    // XCD-aware order. Workgroup ids are dealt round-robin to the 8 XCDs (id % 8), each with its
    // own L2; id -> (xcd j, k-th block of that XCD) -> logical id j * share + k, so every XCD
    // walks a contiguous logical range. Logical order is (batch, tile row, tile col, channel
    // tile, phase) with the channel tiles and phases of one spatial tile consecutive: they read
    // the same input halo, which then comes from L2 rather than HBM.
    const int nz = p.ntiles * (TR ? 4 : 1);
    const int total = p.gx * p.gy * p.N * nz;
    const int bid = (int)blockIdx.x, xj = bid & 7, xk = bid >> 3;
    const int q8 = total >> 3, r8 = total & 7;
    const int lid = xj < r8 ? xj * (q8 + 1) + xk : r8 * (q8 + 1) + (xj - r8) * q8 + xk;
    int rest = lid / nz;
    const int zl = lid - rest * nz;
    const int tx = rest % p.gx;
    rest /= p.gx;
    const int ty = rest % p.gy, bi = rest / p.gy;
    const int phase = TR ? (zl & 3) : 0;
    const int nt = TR ? (zl >> 2) : zl;
    const int gb = nt * NB;
    const int g = gb / p.nblk_g, nb0 = gb - g * p.nblk_g;
    const int ox0 = tx * 16, oy0 = ty * TY;
    // A channel tile of padding blocks only (a narrow tile past cout_g: the packing rounds the
    // blocks up to the layer's default tile) has nothing to compute or store (uniform exit).
    if (nb0 * 16 >= p.cout_g) return;

    int ntap = NTAP;
    int tdy[NTAP], tdx[NTAP];
#pragma unroll
    for (int t = 0; t < NTAP; ++t) {
        if (TR) {
            tdy[t] = p.tap_dy[phase][t];
            tdx[t] = p.tap_dx[phase][t];
        } else {
            tdy[t] = t / KW;
            tdx[t] = t % KW;
        }
    }
    if (TR) ntap = p.ntaps[phase];

    f32x4 acc[CF][PF];
#pragma unroll
    for (int cf = 0; cf < CF; ++cf) {
        const int ocl = (nb0 + wc * CF + cf) * 16 + grp * 4;
        f32x4 b;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            b[i] = (p.bias && ocl + i < p.cout_g) ? p.bias[g * p.cout_g + ocl + i] : 0.0f;
#pragma unroll
        for (int pf = 0; pf < PF; ++pf) acc[cf][pf] = b;
    }

    const int iy0 = TR ? oy0 - 1 : oy0 * S - p.pad_t;
    const int ix0 = TR ? ox0 - 1 : ox0 * S - p.pad_l;
    const T* xg = (const T*)p.x.p + (long long)bi * p.x.bstride;
    const T* wg = (const T*)p.w + phase * p.phase_stride + (long long)bi * p.w_bstride;
    const long long xbase = (long long)p.x.c_off + (long long)g * p.cin_g;

    // LDS slot of halo pixel (hy, hx). Stride-2 halos keep each row's even columns, then its odd
    // ones: a fragment reads every other column (hx = 2 col + kx), which then fall on consecutive
    // 64-byte slots and spread over all banks instead of half of them.
    constexpr int HXE = (HX + 1) / 2;
    auto hslot = [](int hy, int hx) __attribute__((always_inline)) {
        return S == 2 ? hy * HX + ((hx & 1) ? HXE + (hx >> 1) : (hx >> 1)) : hy * HX + hx;
    };
    auto compute = [&](const u32x4* s_halo, const u32x4* s_w) {
        for (int t = 0; t < ntap; ++t) {
            const int ky = tdy[t], kx = tdx[t];
            u32x4 a[CF], b[PF];
#pragma unroll
            for (int cf = 0; cf < CF; ++cf) a[cf] = s_w[((wc * CF + cf) * NTAP + t) * 64 + col * 4 + (grp ^ qswz(col))];
#pragma unroll
            for (int pf = 0; pf < PF; ++pf) {
                const int hy = (wp * PF + pf) * S + ky, hx = col * S + kx, hs = hslot(hy, hx);
                b[pf] = s_halo[hs * 4 + (grp ^ qswz(hs))];
            }
#pragma unroll
            for (int cf = 0; cf < CF; ++cf)
#pragma unroll
                for (int pf = 0; pf < PF; ++pf) Mma<T>::run(acc[cf][pf], a[cf], b[pf]);
        }
    };

    // Halo element offsets of this thread's units (u = tid + i * NT), -1 in the padding; the
    // same for every K chunk.
    long long hoff[HN];
    int hdst[HN];  // LDS unit each halo unit is stored to
#pragma unroll
    for (int i = 0; i < HN; ++i) {
        const int u = tid + i * NT, pix = u >> 2, q = u & 3;
        const int hy = pix / HX, hx = pix - hy * HX;
        const int iy = iy0 + hy, ix = ix0 + hx;
        hoff[i] = (u < HALO_U && iy >= 0 && iy < p.H && ix >= 0 && ix < p.W)
                      ? (long long)iy * p.x.row + (long long)ix * p.x.cs + xbase + q * VEC
                      : -1;
        const int hs = hslot(hy, hx);
        hdst[i] = hs * 4 + (q ^ qswz(hs));
    }
    // One K chunk's halo and weight units into registers. Every load is unconditional, from the
    // unit's address or from a zeroed buffer (padding, channels past cin_g, units past the
    // stage), so all of them are in flight together: a load inside a branch would be waited for
    // before the next one issues.
    auto load_chunk = [&](int chunk, u32x4 (&rh)[HN], u32x4 (&rw)[WN]) __attribute__((always_inline)) {
        const int cl0 = chunk * CK;
#pragma unroll
        for (int i = 0; i < HN; ++i) {
            const int q = (tid + i * NT) & 3;
            const bool ok = hoff[i] >= 0 && cl0 + q * VEC < p.cin_g;
            rh[i] = *(ok ? (const u32x4*)(xg + hoff[i] + cl0) : g_zero_igemm);
        }
        const u32x4* wsrc = (const u32x4*)(wg + ((long long)(g * p.nchunks + chunk) * p.nblk_g + nb0) *
                                                     (long long)(NTAP * 16 * CK));
#pragma unroll
        for (int i = 0; i < WN; ++i) {
            const int u = tid + i * NT;
            rw[i] = *(u < W_U ? wsrc + u : g_zero_igemm);
        }
    };
    auto store_chunk = [&](u32x4* dst, const u32x4 (&rh)[HN], const u32x4 (&rw)[WN]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < HN; ++i) {
            const int u = tid + i * NT;
            u32x4 v = rh[i];
            if (p.relu6_in) v = relu6_vec<T>(v);
            if (u < HALO_U) dst[hdst[i]] = v;
        }
#pragma unroll
        for (int i = 0; i < WN; ++i) {
            const int u = tid + i * NT;
            if (u < W_U) dst[HALO_U + (u & ~3) + ((u & 3) ^ qswz(u >> 2))] = rw[i];
        }
    };

    if constexpr (SG == 1) {
        // The next chunk's loads fly during this chunk's MFMAs.
        u32x4 rh[HN], rw[WN];
        load_chunk(0, rh, rw);
        for (int chunk = 0; chunk < p.nchunks; ++chunk) {
            __syncthreads();
            store_chunk(s_lds, rh, rw);
            __syncthreads();
            if (chunk + 1 < p.nchunks) load_chunk(chunk + 1, rh, rw);
            compute(s_lds, s_lds + HALO_U);
        }
    } else {
        for (int c0 = 0; c0 < p.nchunks; c0 += SG) {
            const int ns = min(SG, p.nchunks - c0);
            u32x4 rh[SG][HN], rw[SG][WN];
#pragma unroll
            for (int s = 0; s < SG; ++s)
                if (s < ns) load_chunk(c0 + s, rh[s], rw[s]);
            __syncthreads();
#pragma unroll
            for (int s = 0; s < SG; ++s)
                if (s < ns) store_chunk(s_lds + s * STG_U, rh[s], rw[s]);
            __syncthreads();
            for (int s = 0; s < ns; ++s) compute(s_lds + s * STG_U, s_lds + s * STG_U + HALO_U);
        }
    }

    if (p.out_mode == OUT_NHWC && p.ps == 1) {
        // Transpose the tile through LDS so that consecutive threads store consecutive channel
        // quads of one position: every position's NB * 16 channels leave as one contiguous run
        // (a lane's accumulator holds 4 channels of one position, 16 lanes apart per position).
        __syncthreads();
        float* so = reinterpret_cast<float*>(s_lds);
#pragma unroll
        for (int cf = 0; cf < CF; ++cf)
#pragma unroll
            for (int pf = 0; pf < PF; ++pf) {
                float* d = so + ((wp * PF + pf) * 16 + col) * OUT_LD + (wc * CF + cf) * 16 + grp * 4;
#pragma unroll
                for (int i = 0; i < 4; ++i) d[i] = acc[cf][pf][i];
            }
        __syncthreads();
        if (nb0 * 16 + NB * 16 <= p.cout_g) {
            // 8 channels per thread and step (all of the tile's channels are real).
            constexpr int QP8 = NB * 2;
#pragma unroll 4
            for (int u = tid; u < TY * 16 * QP8; u += NT) {
                const int pos = u / QP8, c8 = u - pos * QP8;
                const int r = pos >> 4, cx = pos & 15;
                const int oy = TR ? 2 * (oy0 + r) + (phase >> 1) : oy0 + r;
                const int ox = TR ? 2 * (ox0 + cx) + (phase & 1) : ox0 + cx;
                const f32x4 v0 = *reinterpret_cast<const f32x4*>(so + pos * OUT_LD + c8 * 8);
                const f32x4 v1 = *reinterpret_cast<const f32x4*>(so + pos * OUT_LD + c8 * 8 + 4);
                if (oy < p.OH && ox < p.OW) epilogue_store8<T>(p, bi, oy, ox, g * p.cout_g + nb0 * 16 + c8 * 8, v0, v1);
            }
            return;
        }
        constexpr int QP = NB * 4;
        for (int u = tid; u < TY * 16 * QP; u += NT) {
            const int pos = u / QP, cq = u - pos * QP;
            const int r = pos >> 4, cx = pos & 15;
            const int oy = TR ? 2 * (oy0 + r) + (phase >> 1) : oy0 + r;
            const int ox = TR ? 2 * (ox0 + cx) + (phase & 1) : ox0 + cx;
            const int ocl = nb0 * 16 + cq * 4;
            if (oy >= p.OH || ox >= p.OW || ocl >= p.cout_g) continue;
            const f32x4 v = *reinterpret_cast<const f32x4*>(so + pos * OUT_LD + cq * 4);
            epilogue_store<T>(p, bi, oy, ox, g * p.cout_g + ocl, min(4, p.cout_g - ocl), v);
        }
        return;
    }

#pragma unroll
    for (int cf = 0; cf < CF; ++cf) {
        const int ocl = (nb0 + wc * CF + cf) * 16 + grp * 4;
        if (ocl >= p.cout_g) continue;
        const int nvalid = min(4, p.cout_g - ocl);
#pragma unroll
        for (int pf = 0; pf < PF; ++pf) {
            const int r = wp * PF + pf;
            int oy, ox;
            if (TR) {
                oy = 2 * (oy0 + r) + (phase >> 1);
                ox = 2 * (ox0 + col) + (phase & 1);
            } else {
                oy = oy0 + r;
                ox = ox0 + col;
            }
            if (oy >= p.OH || ox >= p.OW) continue;
            epilogue_store<T>(p, bi, oy, ox, g * p.cout_g + ocl, nvalid, acc[cf][pf]);
        }
    }
}

// ---------------------------------------------------------------------------------------------
// fp32 pipelined variant of conv_igemm (dense tile shapes): the input halo and the weight blocks
// of a K stage go global -> LDS with gfx950's direct LDS loads (global_load_lds_dwordx4: lane
// i's 16 bytes land at the wave's LDS base + 16 i, no VGPR staging), double-buffered, so one
// barrier per stage separates the loads of stage k + 1 from the MFMAs of stage k. Padding units
// load from a zeroed device buffer. Numerics are conv_igemm's: bias first, then per K chunk and
// tap the four k = 0..3 MFMAs of each accumulator in order -- issued k-outermost over the
// CF x PF accumulators, so that dependent MFMAs are CF x PF instructions apart.
// ---------------------------------------------------------------------------------------------
__device__ u32x4 g_zero_units[4];

template <int KH, int KW, int S, bool TR, int WC, int WP, int CF, int PF, int SG>
__global__ void __launch_bounds__(WC * WP * 64)
conv_dma_f32(const ConvParams p) {
    using T = float;
    constexpr int NT = WC * WP * 64;
    constexpr int TY = WP * PF;
    constexpr int HY = (TY - 1) * S + KH;
    constexpr int HX = 15 * S + KW;
    constexpr int NTAP = TR ? 4 : KH * KW;
    constexpr int NB = WC * CF;
    constexpr int VEC = 4;
    constexpr int CK = 16;
    constexpr int HALO_U = HY * HX * 4;
    constexpr int W_U = NB * NTAP * 64;
    constexpr int CH_U = HALO_U + W_U;  // one K chunk: halo units, then weight units
    constexpr int STG_U = SG * CH_U;
    constexpr int OUT_LD = NB * 16 + 4;
    constexpr int OUT_U = (TY * 16 * OUT_LD + 3) / 4;
    // Stride-2 stages (a 17 x 33 halo and 4 x 9 weight blocks, 73 KB) are single-buffered: two
    // workgroups per CU then overlap each other's loads, where one double-buffered workgroup left
    // one wave per SIMD.
    constexpr int NBUF = S == 2 ? 1 : 2;
    constexpr int LDS_U = (NBUF * STG_U) > OUT_U ? (NBUF * STG_U) : OUT_U;
    constexpr int HN = (HALO_U + NT - 1) / NT, WN = (W_U + NT - 1) / NT;
    __shared__ u32x4 s_lds[LDS_U];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wc = wave % WC, wp = wave / WC;
    const int col = lane & 15, grp = lane >> 4;

    // Workgroup -> tile: the XCD-aware order of conv_igemm.
    const int nz = p.ntiles * (TR ? 4 : 1);
    const int total = p.gx * p.gy * p.N * nz;
    const int bid = (int)blockIdx.x, xj = bid & 7, xk = bid >> 3;
    const int q8 = total >> 3, r8 = total & 7;
    const int lid = xj < r8 ? xj * (q8 + 1) + xk : r8 * (q8 + 1) + (xj - r8) * q8 + xk;
    int rest = lid / nz;
    const int zl = lid - rest * nz;
    const int tx = rest % p.gx;
    rest /= p.gx;
    const int ty = rest % p.gy, bi = rest / p.gy;
    const int phase = TR ? (zl & 3) : 0;
    const int nt = TR ? (zl >> 2) : zl;
    const int gb = nt * NB;
    const int g = gb / p.nblk_g, nb0 = gb - g * p.nblk_g;
    const int ox0 = tx * 16, oy0 = ty * TY;

    int ntap = NTAP;
    int tdy[NTAP], tdx[NTAP];
#pragma unroll
    for (int t = 0; t < NTAP; ++t) {
        if (TR) {
            tdy[t] = p.tap_dy[phase][t];
            tdx[t] = p.tap_dx[phase][t];
        } else {
            tdy[t] = t / KW;
            tdx[t] = t % KW;
        }
    }
    if (TR) ntap = p.ntaps[phase];

    f32x4 acc[CF][PF];
#pragma unroll
    for (int cf = 0; cf < CF; ++cf) {
        const int ocl = (nb0 + wc * CF + cf) * 16 + grp * 4;
        f32x4 b;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            b[i] = (p.bias && ocl + i < p.cout_g) ? p.bias[g * p.cout_g + ocl + i] : 0.0f;
#pragma unroll
        for (int pf = 0; pf < PF; ++pf) acc[cf][pf] = b;
    }

    const int iy0 = TR ? oy0 - 1 : oy0 * S - p.pad_t;
    const int ix0 = TR ? ox0 - 1 : ox0 * S - p.pad_l;
    const T* xg = (const T*)p.x.p + (long long)bi * p.x.bstride;
    const T* wg = (const T*)p.w + phase * p.phase_stride + (long long)bi * p.w_bstride;
    const long long xbase = (long long)p.x.c_off + (long long)g * p.cin_g;

    // Halo element offset of each of this thread's units (u = tid + i * NT), -1 in the padding,
    // and the first channel of the quad it holds. Stride 2: unit q of halo pixel s holds channel
    // quad q ^ qswz(s); a fragment then reads every other pixel with two lanes per bank quad in
    // each ds_read_b128 pass instead of four. Stride 1 keeps the plain layout.
    long long hoff[HN];
    int hqv[HN];
#pragma unroll
    for (int i = 0; i < HN; ++i) {
        const int u = tid + i * NT, pix = u >> 2, q = u & 3;
        const int hy = pix / HX, hx = pix - hy * HX;
        const int iy = iy0 + hy, ix = ix0 + hx;
        hqv[i] = (S == 2 ? (q ^ qswz(pix)) : q) * VEC;
        hoff[i] = (u < HALO_U && iy >= 0 && iy < p.H && ix >= 0 && ix < p.W)
                      ? (long long)iy * p.x.row + (long long)ix * p.x.cs + xbase + hqv[i]
                      : -1;
    }

    // Direct LDS loads of stage st into buffer buf. Each wave covers whole 64-unit rows of the
    // chunk's layout; its M0 base is the row start, lanes past the end are masked off.
    auto issue = [&](int st, int buf) {
#pragma unroll
        for (int s = 0; s < SG; ++s) {
            const int chunk = st * SG + s;
            if (chunk >= p.nchunks) break;
            const int cl0 = chunk * CK;
            u32x4* dst = s_lds + buf * STG_U + s * CH_U;
#pragma unroll
            for (int i = 0; i < HN; ++i) {
                const int ub = wave * 64 + i * NT;
                if (ub >= HALO_U) break;
                if (ub + lane < HALO_U) {
                    const void* src = (hoff[i] >= 0 && cl0 + hqv[i] < p.cin_g) ? (const void*)(xg + hoff[i] + cl0)
                                                                              : (const void*)g_zero_units;
                    lds_dma16(src, dst + ub);
                }
            }
            const u32x4* wsrc = (const u32x4*)(wg + ((long long)(g * p.nchunks + chunk) * p.nblk_g + nb0) *
                                                        (long long)(NTAP * 16 * CK));
#pragma unroll
            for (int i = 0; i < WN; ++i) {
                const int ub = wave * 64 + i * NT;
                if (ub >= W_U) break;
                if (ub + lane < W_U)
                    lds_dma16(wsrc + ub + lane, dst + HALO_U + ub);
            }
        }
    };

    const int nst = (p.nchunks + SG - 1) / SG;
    issue(0, 0);
    for (int st = 0; st < nst; ++st) {
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's loads of stage st are in LDS
        __syncthreads();                     // ... and every other wave's
        if (NBUF == 2 && st + 1 < nst) issue(st + 1, (st + 1) & 1);
        const u32x4* sb = s_lds + (NBUF == 2 ? (st & 1) : 0) * STG_U;
        auto stage = [&](auto relu6) {
#pragma unroll
            for (int s = 0; s < SG; ++s) {
                if (st * SG + s >= p.nchunks) break;
                const u32x4* s_halo = sb + s * CH_U;
                const u32x4* s_w = s_halo + HALO_U;
                for (int t = 0; t < ntap; ++t) {
                    const int ky = tdy[t], kx = tdx[t];
                    u32x4 a[CF], b[PF];
#pragma unroll
                    for (int cf = 0; cf < CF; ++cf) a[cf] = s_w[((wc * CF + cf) * NTAP + t) * 64 + col * 4 + grp];
#pragma unroll
                    for (int pf = 0; pf < PF; ++pf) {
                        const int hy = (wp * PF + pf) * S + ky, hx = col * S + kx, hs = hy * HX + hx;
                        b[pf] = s_halo[hs * 4 + (S == 2 ? (grp ^ qswz(hs)) : grp)];
                        if constexpr (decltype(relu6)::value) b[pf] = relu6_vec<T>(b[pf]);
                    }
#pragma unroll
                    for (int k = 0; k < 4; ++k)
#pragma unroll
                        for (int cf = 0; cf < CF; ++cf)
#pragma unroll
                            for (int pf = 0; pf < PF; ++pf)
                                acc[cf][pf] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                                    __builtin_bit_cast(f32x4, a[cf])[k], __builtin_bit_cast(f32x4, b[pf])[k],
                                    acc[cf][pf], 0, 0, 0);
                }
            }
        };
        if (p.relu6_in) stage(std::true_type{});
        else stage(std::false_type{});
        if (NBUF == 1 && st + 1 < nst) {
            __syncthreads();  // every wave is done with the buffer
            issue(st + 1, 0);
        }
    }

    if (p.out_mode == OUT_NHWC && p.ps == 1) {
        __syncthreads();
        float* so = reinterpret_cast<float*>(s_lds);
#pragma unroll
        for (int cf = 0; cf < CF; ++cf)
#pragma unroll
            for (int pf = 0; pf < PF; ++pf) {
                float* d = so + ((wp * PF + pf) * 16 + col) * OUT_LD + (wc * CF + cf) * 16 + grp * 4;
#pragma unroll
                for (int i = 0; i < 4; ++i) d[i] = acc[cf][pf][i];
            }
        __syncthreads();
        if (nb0 * 16 + NB * 16 <= p.cout_g) {
            // 8 channels per thread and step (all of the tile's channels are real).
            constexpr int QP8 = NB * 2;
#pragma unroll 4
            for (int u = tid; u < TY * 16 * QP8; u += NT) {
                const int pos = u / QP8, c8 = u - pos * QP8;
                const int r = pos >> 4, cx = pos & 15;
                const int oy = TR ? 2 * (oy0 + r) + (phase >> 1) : oy0 + r;
                const int ox = TR ? 2 * (ox0 + cx) + (phase & 1) : ox0 + cx;
                const f32x4 v0 = *reinterpret_cast<const f32x4*>(so + pos * OUT_LD + c8 * 8);
                const f32x4 v1 = *reinterpret_cast<const f32x4*>(so + pos * OUT_LD + c8 * 8 + 4);
                if (oy < p.OH && ox < p.OW) epilogue_store8<T>(p, bi, oy, ox, g * p.cout_g + nb0 * 16 + c8 * 8, v0, v1);
            }
            return;
        }
        constexpr int QP = NB * 4;
        for (int u = tid; u < TY * 16 * QP; u += NT) {
            const int pos = u / QP, cq = u - pos * QP;
            const int r = pos >> 4, cx = pos & 15;
            const int oy = TR ? 2 * (oy0 + r) + (phase >> 1) : oy0 + r;
            const int ox = TR ? 2 * (ox0 + cx) + (phase & 1) : ox0 + cx;
            const int ocl = nb0 * 16 + cq * 4;
            if (oy >= p.OH || ox >= p.OW || ocl >= p.cout_g) continue;
            const f32x4 v = *reinterpret_cast<const f32x4*>(so + pos * OUT_LD + cq * 4);
            epilogue_store<T>(p, bi, oy, ox, g * p.cout_g + ocl, min(4, p.cout_g - ocl), v);
        }
        return;
    }

#pragma unroll
    for (int cf = 0; cf < CF; ++cf) {
        const int ocl = (nb0 + wc * CF + cf) * 16 + grp * 4;
        if (ocl >= p.cout_g) continue;
        const int nvalid = min(4, p.cout_g - ocl);
#pragma unroll
        for (int pf = 0; pf < PF; ++pf) {
            const int r = wp * PF + pf;
            const int oy = TR ? 2 * (oy0 + r) + (phase >> 1) : oy0 + r;
            const int ox = TR ? 2 * (ox0 + col) + (phase & 1) : ox0 + col;
            if (oy >= p.OH || ox >= p.OW) continue;
            epilogue_store<T>(p, bi, oy, ox, g * p.cout_g + ocl, nvalid, acc[cf][pf]);
        }
    }
}

// ---------------------------------------------------------------------------------------------
// Stride-2 transposed conv (3x3 kernel) with the four output phases of a tile in one
// workgroup. The phase-per-workgroup form stages a halo and a weight block per K chunk for
// 1, 2, 2 or 4 taps; here the 9 taps of all phases share one staged halo and one 9-tap weight
// block, so a K chunk carries as much matrix work as a 3x3 conv. Each wave accumulates its
// CF x PF tile for all four phases (acc[4][CF][PF]); the stage pipeline is conv_dma_f32's
// (direct global -> LDS loads, double-buffered, one barrier per stage), for every storage type.
// Per output the products are summed exactly as in the phase-per-workgroup kernel: bias, then
// per K chunk the phase's taps in table order, k ascending within a tap. The phases' tap counts
// are template parameters (1, 2, 2, 4 for padding 1; 4, 2, 2, 1 for padding 0 or 2), so the tap
// loops unroll and each tap's fragment reads overlap the previous tap's MFMAs.
// ---------------------------------------------------------------------------------------------
template <typename T, int N0, int N1, int N2, int N3>
__global__ void __launch_bounds__(512)
conv_tr_merged(const ConvParams p) {
    // 16-bit weights come packed with unit q of each 16-row block's row r at q ^ qswz(r) (the
    // launcher's merged packing), so the fragment reads are conflict-free; f32 keeps the plain
    // layout (under the swizzled addressing the compiler renamed this kernel's f32 MFMA chains).
    auto wswz = [](int r) __attribute__((always_inline)) { return sizeof(T) == 2 ? qswz(r) : 0; };
    constexpr int WC = 2, WP = 4, CF = 2, PF = 4;
    constexpr int NT = WC * WP * 64;
    constexpr int TY = WP * PF;
    constexpr int HY = TY + 2, HX = 18;
    constexpr int NTALL = TR_MERGED_TAPS;
    constexpr int NB = WC * CF;
    static_assert(NB == TR_MERGED_NB, "packing block count");
    constexpr int VEC = 16 / (int)sizeof(T);
    constexpr int CK = 4 * VEC;
    constexpr int HALO_U = HY * HX * 4;
    constexpr int W_U = NB * NTALL * 64;
    constexpr int CH_U = HALO_U + W_U;
    constexpr int OUT_LD = NB * 16 + 4;
    constexpr int OUT_U = (TY * 16 * OUT_LD + 3) / 4;
    constexpr int LDS_U = (2 * CH_U) > OUT_U ? (2 * CH_U) : OUT_U;
    constexpr int HN = (HALO_U + NT - 1) / NT, WN = (W_U + NT - 1) / NT;
    __shared__ u32x4 s_lds[LDS_U];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wc = wave % WC, wp = wave / WC;
    const int col = lane & 15, grp = lane >> 4;

    const int nz = p.ntiles;
    const int total = p.gx * p.gy * p.N * nz;
    const int bid = (int)blockIdx.x, xj = bid & 7, xk = bid >> 3;
    const int q8 = total >> 3, r8 = total & 7;
    const int lid = xj < r8 ? xj * (q8 + 1) + xk : r8 * (q8 + 1) + (xj - r8) * q8 + xk;
    int rest = lid / nz;
    const int zl = lid - rest * nz;
    const int tx = rest % p.gx;
    rest /= p.gx;
    const int ty = rest % p.gy, bi = rest / p.gy;
    const int nb0 = zl * NB;
    const int ox0 = tx * 16, oy0 = ty * TY;

    f32x4 acc[4][CF][PF];
#pragma unroll
    for (int cf = 0; cf < CF; ++cf) {
        const int ocl = (nb0 + wc * CF + cf) * 16 + grp * 4;
        f32x4 b;
#pragma unroll
        for (int i = 0; i < 4; ++i) b[i] = (p.bias && ocl + i < p.cout_g) ? p.bias[ocl + i] : 0.0f;
#pragma unroll
        for (int ph = 0; ph < 4; ++ph)
#pragma unroll
            for (int pf = 0; pf < PF; ++pf) acc[ph][cf][pf] = b;
    }

    const int iy0 = oy0 - 1, ix0 = ox0 - 1;
    const T* xg = (const T*)p.x.p + (long long)bi * p.x.bstride + p.x.c_off;
    const u32x4* wg = (const u32x4*)p.w + (long long)nb0 * (NTALL * 64);
    const long long wchunk = (long long)p.nblk_g * (NTALL * 64);

    long long hoff[HN];
#pragma unroll
    for (int i = 0; i < HN; ++i) {
        const int u = tid + i * NT, pix = u >> 2, q = u & 3;
        const int hy = pix / HX, hx = pix - hy * HX;
        const int iy = iy0 + hy, ix = ix0 + hx;
        hoff[i] = (u < HALO_U && iy >= 0 && iy < p.H && ix >= 0 && ix < p.W)
                      ? (long long)iy * p.x.row + (long long)ix * p.x.cs + q * VEC
                      : -1;
    }
    const int qv = (tid & 3) * VEC;

    // Tap tables in registers (compile-time indices below), so that the kernel argument block
    // is never indexed at run time.
    static_assert(N0 + N1 + N2 + N3 == NTALL, "tap counts");
    constexpr int NTP[4] = {N0, N1, N2, N3};
    constexpr int BASE[4] = {0, N0, N0 + N1, N0 + N1 + N2};
    int tdy[4][4], tdx[4][4];
#pragma unroll
    for (int ph = 0; ph < 4; ++ph)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            tdy[ph][t] = t < NTP[ph] ? p.tap_dy[ph][t] : 0;
            tdx[ph][t] = t < NTP[ph] ? p.tap_dx[ph][t] : 0;
        }
    const int nchunks = p.nchunks, cin_g = p.cin_g;

    auto issue = [&](int chunk, int buf) __attribute__((always_inline)) {
        const int cl0 = chunk * CK;
        u32x4* dst = s_lds + buf * CH_U;
#pragma unroll
        for (int i = 0; i < HN; ++i) {
            const int ub = wave * 64 + i * NT;
            if (ub >= HALO_U) break;
            if (ub + lane < HALO_U) {
                const void* src = (hoff[i] >= 0 && cl0 + qv < cin_g) ? (const void*)(xg + hoff[i] + cl0)
                                                                      : (const void*)g_zero_units;
                lds_dma16(src, dst + ub);
            }
        }
        const u32x4* wsrc = wg + chunk * wchunk;
#pragma unroll
        for (int i = 0; i < WN; ++i) {
            const int ub = wave * 64 + i * NT;
            if (ub >= W_U) break;
            if (ub + lane < W_U)
                lds_dma16(wsrc + ub + lane, dst + HALO_U + ub);
        }
    };


    issue(0, 0);
    for (int c = 0; c < nchunks; ++c) {
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's loads of chunk c are in LDS
        __syncthreads();                     // ... and every other wave's
        if (c + 1 < nchunks) issue(c + 1, (c + 1) & 1);
        const u32x4* s_halo = s_lds + (c & 1) * CH_U;
        const u32x4* s_w = s_halo + HALO_U;
        auto phase_taps = [&](auto phc) __attribute__((always_inline)) {
            constexpr int ph = decltype(phc)::value;
#pragma unroll
            for (int t = 0; t < NTP[ph]; ++t) {
                const int e = BASE[ph] + t;
                const int dy = tdy[ph][t], dx = tdx[ph][t];
                u32x4 a[CF], b[PF];
#pragma unroll
                for (int cf = 0; cf < CF; ++cf) a[cf] = s_w[((wc * CF + cf) * NTALL + e) * 64 + col * 4 + (grp ^ wswz(col))];
#pragma unroll
                for (int pf = 0; pf < PF; ++pf) {
                    b[pf] = s_halo[((wp * PF + pf + dy) * HX + col + dx) * 4 + grp];
                }
                if constexpr (sizeof(T) == 4) {
#pragma unroll
                    for (int k = 0; k < 4; ++k)
#pragma unroll
                        for (int cf = 0; cf < CF; ++cf)
#pragma unroll
                            for (int pf = 0; pf < PF; ++pf)
                                acc[ph][cf][pf] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                                    __builtin_bit_cast(f32x4, a[cf])[k], __builtin_bit_cast(f32x4, b[pf])[k],
                                    acc[ph][cf][pf], 0, 0, 0);
                } else {
#pragma unroll
                    for (int cf = 0; cf < CF; ++cf)
#pragma unroll
                        for (int pf = 0; pf < PF; ++pf) Mma<T>::run(acc[ph][cf][pf], a[cf], b[pf]);
                }
            }
        };
        phase_taps(std::integral_constant<int, 0>{});
        phase_taps(std::integral_constant<int, 1>{});
        phase_taps(std::integral_constant<int, 2>{});
        phase_taps(std::integral_constant<int, 3>{});
    }

    // One phase at a time through the LDS transpose (NHWC output without pixel shuffle; the
    // launcher sends every other epilogue to the phase-per-workgroup kernel).
    float* so = reinterpret_cast<float*>(s_lds);
    auto put = [&](const f32x4 (&a)[CF][PF]) __attribute__((always_inline)) {
#pragma unroll
        for (int cf = 0; cf < CF; ++cf)
#pragma unroll
            for (int pf = 0; pf < PF; ++pf) {
                float* d = so + ((wp * PF + pf) * 16 + col) * OUT_LD + (wc * CF + cf) * 16 + grp * 4;
#pragma unroll
                for (int i = 0; i < 4; ++i) d[i] = a[cf][pf][i];
            }
    };
    for (int ph = 0; ph < 4; ++ph) {
        __syncthreads();
        if (ph == 0) put(acc[0]);
        else if (ph == 1) put(acc[1]);
        else if (ph == 2) put(acc[2]);
        else put(acc[3]);
        __syncthreads();
        const int py = ph >> 1, px = ph & 1;
        if (epilogue_simple(p) && nb0 * 16 + NB * 16 <= p.cout_g) {
            // 8 channels per thread and step (all of the tile's channels are real).
            constexpr int QP8 = NB * 2;
#pragma unroll 4
            for (int u = tid; u < TY * 16 * QP8; u += NT) {
                const int pos = u / QP8, c8 = u - pos * QP8;
                const int r = pos >> 4, cx = pos & 15;
                const int oy = 2 * (oy0 + r) + py, ox = 2 * (ox0 + cx) + px;
                const f32x4 v0 = *reinterpret_cast<const f32x4*>(so + pos * OUT_LD + c8 * 8);
                const f32x4 v1 = *reinterpret_cast<const f32x4*>(so + pos * OUT_LD + c8 * 8 + 4);
                if (oy < p.OH && ox < p.OW) epilogue_store8<T>(p, bi, oy, ox, nb0 * 16 + c8 * 8, v0, v1);
            }
        } else {
            constexpr int QP = NB * 4;
            for (int u = tid; u < TY * 16 * QP; u += NT) {
                const int pos = u / QP, cq = u - pos * QP;
                const int r = pos >> 4, cx = pos & 15;
                const int oy = 2 * (oy0 + r) + py, ox = 2 * (ox0 + cx) + px;
                const int ocl = nb0 * 16 + cq * 4;
                if (oy >= p.OH || ox >= p.OW || ocl >= p.cout_g) continue;
                const f32x4 v = *reinterpret_cast<const f32x4*>(so + pos * OUT_LD + cq * 4);
                epilogue_store<T>(p, bi, oy, ox, ocl, min(4, p.cout_g - ocl), v);
            }
        }
    }
}

hipError_t launch_conv_tr_merged(int dtype, const ConvParams& p0, hipStream_t s) {
    ConvParams p = p0;
    if (p.groups != 1 || p.ntiles * TR_MERGED_NB != p.nblk_g || p.N < 1 || p.N > MAXB || p.out_mode != OUT_NHWC ||
        p.ps != 1 || p.relu6_in)
        return hipErrorInvalidValue;
    if (p.ntaps[0] + p.ntaps[1] + p.ntaps[2] + p.ntaps[3] != TR_MERGED_TAPS) return hipErrorInvalidValue;
    for (int ph = 0; ph < 4; ++ph)
        for (int t = 0; t < p.ntaps[ph]; ++t)
            if (p.tap_dy[ph][t] < 0 || p.tap_dy[ph][t] > 2 || p.tap_dx[ph][t] < 0 || p.tap_dx[ph][t] > 2)
                return hipErrorInvalidValue;
    p.gx = ((p.OW + 1) / 2 + 15) / 16;
    p.gy = ((p.OH + 1) / 2 + 15) / 16;
    const long long total = (long long)p.gx * p.gy * p.N * p.ntiles;
    if (total <= 0 || total > (1ll << 30)) return hipErrorInvalidValue;
    const bool pad1 = p.ntaps[0] == 1 && p.ntaps[1] == 2 && p.ntaps[2] == 2 && p.ntaps[3] == 4;
    const bool pad02 = p.ntaps[0] == 4 && p.ntaps[1] == 2 && p.ntaps[2] == 2 && p.ntaps[3] == 1;
    if (!pad1 && !pad02) return hipErrorInvalidValue;
    const dim3 grid((unsigned)total), block(512);
#define ZJAI_TRM(TY)                                                                                 \
    do {                                                                                             \
        if (pad1) hipLaunchKernelGGL((conv_tr_merged<TY, 1, 2, 2, 4>), grid, block, 0, s, p);       \
        else hipLaunchKernelGGL((conv_tr_merged<TY, 4, 2, 2, 1>), grid, block, 0, s, p);            \
    } while (0)
    switch (dtype) {
        case DT_F32: ZJAI_TRM(float); break;
        case DT_F16: ZJAI_TRM(_Float16); break;
        case DT_BF16: ZJAI_TRM(__bf16); break;
        default: return hipErrorInvalidValue;
    }
#undef ZJAI_TRM
    return hipGetLastError();
}

bool conv_tr_merged_taps_supported(const int (&ntaps)[4]) {
    return (ntaps[0] == 1 && ntaps[1] == 2 && ntaps[2] == 2 && ntaps[3] == 4) ||
           (ntaps[0] == 4 && ntaps[1] == 2 && ntaps[2] == 2 && ntaps[3] == 1);
}

// ---------------------------------------------------------------------------------------------
// Narrow transposed convolution (stride 2, at most 8 output channels): the last synthesis layers
// (HOP luma 128 -> 1, chroma 64 -> 8). An MFMA tile would leave at least half of its 16 or 32
// output rows idle, so these run on the vector ALUs: one thread per phase-grid position (y', x')
// computes its 2x2 output phases for every output channel. Per output: acc = bias, then for each
// input channel ascending and each reaching tap in (ky, kx) order acc = fma(w, x, acc) -- the
// reference's convT order (src/nn/reference.rs:155-236), so in f32 the result equals the oracle
// bit for bit. Per chunk of 16 input channels a workgroup stages its (TYN + 2) x (TXN + 2) input
// halo in LDS channel-major, so consecutive threads read consecutive words.
// wn: [cin][phase][tap][COUT] f32 (weights already rounded to the storage type).
template <typename T, int COUT>
__global__ void __launch_bounds__(256)
k_convT_narrow(const ConvParams p, const float* __restrict__ wn, int cin) {
    constexpr int TXN = 64, TYN = 4, HXN = TXN + 2, HYN = TYN + 2, CKN = 16;
    constexpr int HP = HXN * HYN;
    __shared__ float s_x[CKN * HP];
    __shared__ float s_w[4 * 4 * CKN * COUT];
    const int gw = (p.OW + 1) / 2, gh = (p.OH + 1) / 2;
    const int gx = (gw + TXN - 1) / TXN, gy = (gh + TYN - 1) / TYN;
    // XCD-aware order: workgroups go to the 8 XCDs round-robin, so workgroup q takes tile
    // (q % 8) * (gridDim.x / 8) + q / 8 and each XCD runs one contiguous band of tile rows,
    // whose shared halo rows then meet in its L2. The grid is a multiple of 8; extra
    // workgroups exit (uniformly, before any barrier).
    int bid = (int)((blockIdx.x % 8) * (gridDim.x / 8) + blockIdx.x / 8);
    if (bid >= gx * gy * p.N) return;
    const int tx = bid % gx;
    bid /= gx;
    const int ty = bid % gy, bi = bid / gy;
    const int tid = threadIdx.x, r = tid / TXN, c = tid % TXN;
    const int y0 = ty * TYN, x0 = tx * TXN;
    const T* xg = (const T*)p.x.p + (long long)bi * p.x.bstride;

    int nt[4], tdy[4][4], tdx[4][4];
#pragma unroll
    for (int ph = 0; ph < 4; ++ph) {
        nt[ph] = p.ntaps[ph];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            tdy[ph][t] = p.tap_dy[ph][t];
            tdx[ph][t] = p.tap_dx[ph][t];
        }
    }
    float acc[4][COUT];
#pragma unroll
    for (int ph = 0; ph < 4; ++ph)
#pragma unroll
        for (int oc = 0; oc < COUT; ++oc) acc[ph][oc] = (p.bias && oc < p.cout_g) ? p.bias[oc] : 0.0f;

    for (int c0 = 0; c0 < cin; c0 += CKN) {
        __syncthreads();
        // Halo: pixel (hy, hx) <- input (y0 - 1 + hy, x0 - 1 + hx); 4 channels per thread step.
        for (int u = tid; u < HP * (CKN / 4); u += 256) {
            const int pix = u / (CKN / 4), q = u - pix * (CKN / 4);
            const int hy = pix / HXN, hx = pix - hy * HXN;
            const int iy = y0 - 1 + hy, ix = x0 - 1 + hx, ch = c0 + 4 * q;
            f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
            if (iy >= 0 && iy < p.H && ix >= 0 && ix < p.W && ch < cin) {
                v = load4<T>(xg + (long long)iy * p.x.row + (long long)ix * p.x.cs + p.x.c_off + ch);
                if (p.relu6_in) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        float e = v[i];
                        e = e < 0.0f ? 0.0f : e;
                        v[i] = e > 6.0f ? 6.0f : e;
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) s_x[(4 * q + i) * HP + pix] = v[i];
        }
        for (int u = tid; u < 4 * 4 * CKN * COUT; u += 256) {
            const int oc = u % COUT, k = (u / COUT) % CKN, pt = u / (COUT * CKN);
            s_w[u] = c0 + k < cin ? wn[((long long)(c0 + k) * 16 + pt) * COUT + oc] : 0.0f;
        }
        __syncthreads();
        const int kn = min(CKN, cin - c0);
        for (int k = 0; k < kn; ++k) {
            const float* sx = s_x + k * HP;
#pragma unroll
            for (int ph = 0; ph < 4; ++ph)
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    if (t >= nt[ph]) break;
                    const float x = sx[(r + tdy[ph][t]) * HXN + c + tdx[ph][t]];
                    const float* w = s_w + ((ph * 4 + t) * CKN + k) * COUT;
#pragma unroll
                    for (int oc = 0; oc < COUT; ++oc) acc[ph][oc] = fmaf(w[oc], x, acc[ph][oc]);
                }
        }
    }
    const int yq = y0 + r, xq = x0 + c;
#pragma unroll
    for (int ph = 0; ph < 4; ++ph) {
        const int oy = 2 * yq + (ph >> 1), ox = 2 * xq + (ph & 1);
        if (oy >= p.OH || ox >= p.OW) continue;
#pragma unroll
        for (int oc0 = 0; oc0 < COUT; oc0 += 4) {
            if (oc0 >= p.cout_g) break;
            f32x4 v;
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = oc0 + i < COUT ? acc[ph][min(oc0 + i, COUT - 1)] : 0.0f;
            epilogue_store<T>(p, bi, oy, ox, oc0, min(4, p.cout_g - oc0), v);
        }
    }
}

// The same layer for the 3x3 kernel with padding 1 (the synthesis nets' conv3x3_t): its taps
// are fixed, phase (py, px) reading input (y' + a, x' + b) for a <= py, b <= px, so a position
// needs only the 2 x 2 input neighbourhood (y', x') .. (y' + 1, x' + 1). A workgroup of 256
// threads takes 8 x 32 positions; per chunk of 64 bytes of input channels (16 f32 or 32
// f16 / bf16) the 9 x 33 input halo goes global -> LDS with direct loads (halo overhead 1.16x),
// double-buffered in 38 KB, so that four workgroups share a CU and one's loads fly while the
// others run their FMAs (128-byte chunks, 76 KB and two workgroups per CU: f32 127 -> 107 us
// per config-5 launch), 16-byte slots XOR-swizzled by pixel so that each thread's 16-byte
// neighbour reads are free of bank conflicts. Weights come through scalar loads ([cin][phase][tap][COUT], uniform). Against the
// generic kernel on HOP luma's 128 -> 1 layer (862 x 862 positions): f32 153 vs 270 us, bf16
// 122 vs 226 us. FMA order
// per output is the generic kernel's (input channel ascending, then the phase's taps in
// (ky, kx) order), so the results are identical to it bit for bit.
__device__ u32x4 g_zero_unitsT[4];  // 64 zero bytes: the source of halo pixels off the map

template <typename T>
__device__ __forceinline__ void unpack16(u32x4 u, float (&v)[16 / sizeof(T)]) {
    if constexpr (sizeof(T) == 4) {
        const f32x4 f = __builtin_bit_cast(f32x4, u);
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = f[i];
    } else {
        typedef T t8 __attribute__((ext_vector_type(8)));
        const t8 h = __builtin_bit_cast(t8, u);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = (float)h[i];
    }
}

template <typename T, int COUT>
__global__ void __launch_bounds__(256)
k_convT3_narrow(const ConvParams p, const float* __restrict__ wn, int cin) {
    constexpr int TY = 8, TX = 32, HX = TX + 1, HY = TY + 1, HPIX = HX * HY;
    constexpr int VEC = 16 / (int)sizeof(T);
    constexpr int CPU = 4;                            // 16-byte units per pixel and chunk
    constexpr int HALO_U = HPIX * CPU;                // [pixel][CPU swizzled 16-byte slots]
    constexpr int HN = (HALO_U + 255) / 256;
    __shared__ u32x4 s_halo[2 * HALO_U];
    const int gw = (p.OW + 1) / 2, gh = (p.OH + 1) / 2;
    const int gx = (gw + TX - 1) / TX, gy = (gh + TY - 1) / TY;
    // XCD-aware order (k_convT_narrow's): each XCD takes one contiguous band of tiles.
    int bid = (int)((blockIdx.x % 8) * (gridDim.x / 8) + blockIdx.x / 8);
    if (bid >= gx * gy * p.N) return;
    const int tx = bid % gx;
    bid /= gx;
    const int ty = bid % gy, bi = bid / gy;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = tid / TX, c = tid % TX;
    const int y0 = ty * TY, x0 = tx * TX;
    const T* xg = (const T*)p.x.p + (long long)bi * p.x.bstride + p.x.c_off;

    float acc[4][COUT];
#pragma unroll
    for (int ph = 0; ph < 4; ++ph)
#pragma unroll
        for (int oc = 0; oc < COUT; ++oc) acc[ph][oc] = (p.bias && oc < p.cout_g) ? p.bias[oc] : 0.0f;

    // Halo unit U = pixel * CPU + slot holds the pixel's 16-byte unit slot ^ ((pixel / 4) % 4):
    // the 16 lanes of each ds_read_b128 pass (32 neighbouring pixels per wave row) then sit on
    // distinct bank quads for any first pixel.
    long long hoff[HN];
#pragma unroll
    for (int i = 0; i < HN; ++i) {
        const int U = wave * 64 + i * 256 + lane, pix = U >> 2, slot = U & 3;
        const int hy = pix / HX, hx = pix - hy * HX;
        const int iy = y0 + hy, ix = x0 + hx;
        hoff[i] = (U < HALO_U && iy < p.H && ix < p.W)
                      ? (long long)iy * p.x.row + (long long)ix * p.x.cs + (slot ^ ((pix >> 2) & 3)) * VEC
                      : -1;
    }
    auto issue = [&](int chunk, int buf) __attribute__((always_inline)) {
        const long long c0 = (long long)chunk * CPU * VEC;
#pragma unroll
        for (int i = 0; i < HN; ++i) {
            const int ub = wave * 64 + i * 256;
            if (ub >= HALO_U) break;
            if (ub + lane < HALO_U) {
                const void* src = hoff[i] >= 0 ? (const void*)(xg + hoff[i] + c0) : (const void*)g_zero_unitsT;
                lds_dma16(src, s_halo + buf * HALO_U + ub);
            }
        }
    };
    int npix[4];  // neighbours (y' + a, x' + b), index 2a + b
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) npix[2 * a + b] = (r + a) * HX + c + b;

    const int nch = cin / (CPU * VEC);
    issue(0, 0);
    for (int ch = 0; ch < nch; ++ch) {
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's loads of chunk ch are in LDS
        __syncthreads();                     // ... and every other wave's
        if (ch + 1 < nch) issue(ch + 1, (ch + 1) & 1);
        const u32x4* hb = s_halo + (ch & 1) * HALO_U;
#pragma unroll 2
        for (int q = 0; q < CPU; ++q) {
            float x[4][VEC];
#pragma unroll
            for (int n = 0; n < 4; ++n) {
                const int pix = npix[n];
                unpack16<T>(hb[pix * CPU + (q ^ ((pix >> 2) & 3))], x[n]);
                if (p.relu6_in) {
#pragma unroll
                    for (int i = 0; i < VEC; ++i) {
                        float e = x[n][i];
                        e = e < 0.0f ? 0.0f : e;
                        x[n][i] = e > 6.0f ? 6.0f : e;
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < VEC; ++i) {
                const float* w = wn + (long long)((ch * CPU + q) * VEC + i) * 16 * COUT;
                // Phase taps in (ky, kx) order: (0,0): x00; (0,1): x01, x00; (1,0): x10, x00;
                // (1,1): x11, x10, x01, x00.
#pragma unroll
                for (int oc = 0; oc < COUT; ++oc) {
                    acc[0][oc] = fmaf(w[0 * COUT + oc], x[0][i], acc[0][oc]);
                    acc[1][oc] = fmaf(w[4 * COUT + oc], x[1][i], acc[1][oc]);
                    acc[1][oc] = fmaf(w[5 * COUT + oc], x[0][i], acc[1][oc]);
                    acc[2][oc] = fmaf(w[8 * COUT + oc], x[2][i], acc[2][oc]);
                    acc[2][oc] = fmaf(w[9 * COUT + oc], x[0][i], acc[2][oc]);
                    acc[3][oc] = fmaf(w[12 * COUT + oc], x[3][i], acc[3][oc]);
                    acc[3][oc] = fmaf(w[13 * COUT + oc], x[2][i], acc[3][oc]);
                    acc[3][oc] = fmaf(w[14 * COUT + oc], x[1][i], acc[3][oc]);
                    acc[3][oc] = fmaf(w[15 * COUT + oc], x[0][i], acc[3][oc]);
                }
            }
        }
    }
    const int yq = y0 + r, xq = x0 + c;
#pragma unroll
    for (int ph = 0; ph < 4; ++ph) {
        const int oy = 2 * yq + (ph >> 1), ox = 2 * xq + (ph & 1);
        if (oy >= p.OH || ox >= p.OW) continue;
#pragma unroll
        for (int oc0 = 0; oc0 < COUT; oc0 += 4) {
            if (oc0 >= p.cout_g) break;
            f32x4 v;
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = oc0 + i < COUT ? acc[ph][min(oc0 + i, COUT - 1)] : 0.0f;
            epilogue_store<T>(p, bi, oy, ox, oc0, min(4, p.cout_g - oc0), v);
        }
    }
}

// ---------------------------------------------------------------------------------------------
// 16-bit 3x3 stride-2 transposed convs with at most 8 outputs and 64 or 128 input channels (the
// last synthesis layers: HOP luma 128 -> 1, HOP chroma 64 -> 8) on the matrix cores. Output phase
// (py, px) of phase-grid position (y', x') reads only the 2 x 2 input neighbourhood
// (y' + a, x' + b), so the layer is one GEMM per position: K = 4 neighbours x CIN, M = 4 phases x
// COUTP rows (row R = phase * COUTP + output; a phase's weight for a neighbour it does not read
// is zero), N = positions. 16x16x32 MFMAs with the weights as A (MB 16-row blocks, packed
// [CIN / 32][4][MB][16][32], held in registers) and the halo as B. A workgroup (4 waves) takes
// 8 x TX positions (TX = 32, or 16 for 128 input channels: a 39 KB halo, four workgroups per CU
// instead of two, so more halo loads fly while other workgroups compute) and stages its whole
// 9 x (TX + 1)-pixel input halo, every channel, in one round trip (direct LDS loads of whole 128- or 256-byte pixels, 16-byte slots XORed by pixel so that a
// fragment's 16 pixels spread over the banks): the layer is one HBM read of its input, and its
// 9 FMAs per input channel and output on the vector ALUs become one fragment read per 32
// channels. Products of 16-bit operands are exact in f32, so the result differs from the vector
// kernel's (input channel, tap) FMA chain by the summation order only, before the final rounding
// to the storage type.
template <typename T, int COUTP, int CIN, int TX>
__global__ void __launch_bounds__(256)
k_convT3_mfma(const ConvParams p, const u32x4* __restrict__ wm) {
    constexpr int MB = (4 * COUTP + 15) / 16;  // 16-row blocks of (phase, output) rows
    constexpr int TY = 8, HX = TX + 1, HY = TY + 1, HPIX = HX * HY;
    constexpr int NJ = TX / 8;                 // 16-position blocks per wave (two tile rows)
    constexpr int BR = TX / 16;                // blocks per tile row
    static_assert(TX == 16 || TX == 32, "tile width");
    constexpr int SL = CIN / 8;                // 16-byte slots per pixel
    constexpr int HALO_U = HPIX * SL;
    constexpr int HN = (HALO_U + 255) / 256;
    constexpr int KC = CIN / 32;               // 32-channel K steps per neighbour
    constexpr int WF = KC * 4 * MB;            // weight fragments
    static_assert(sizeof(T) == 2 && (CIN == 64 || CIN == 128), "16-bit, 64 or 128 input channels");
    __shared__ u32x4 s_halo[HALO_U];
    // Slot swizzle: consecutive pixels' same slot lands in different banks.
    auto swz = [](int pix) { return SL == 16 ? (pix & 15) : ((pix >> 1) & 7); };
    const int gw = (p.OW + 1) / 2, gh = (p.OH + 1) / 2;
    const int gx = (gw + TX - 1) / TX, gy = (gh + TY - 1) / TY;
    int bid = (int)((blockIdx.x % 8) * (gridDim.x / 8) + blockIdx.x / 8);
    if (bid >= gx * gy * p.N) return;
    const int tx = bid % gx;
    bid /= gx;
    const int ty = bid % gy, bi = bid / gy;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int y0 = ty * TY, x0 = tx * TX;
    const T* xg = (const T*)p.x.p + (long long)bi * p.x.bstride + p.x.c_off;

    // The whole halo: unit U = pixel * SL + slot holds the pixel's 16-byte unit slot ^ swz(pixel).
#pragma unroll
    for (int i = 0; i < HN; ++i) {
        const int ub = wave * 64 + i * 256;
        if (ub >= HALO_U) break;
        const int U = ub + lane, pix = U / SL, slot = U % SL;
        const int hy = pix / HX, hx = pix - hy * HX;
        const int iy = y0 + hy, ix = x0 + hx;
        const void* src = (U < HALO_U && iy < p.H && ix < p.W)
                              ? (const void*)(xg + (long long)iy * p.x.row + (long long)ix * p.x.cs + (slot ^ swz(pix)) * 8)
                              : (const void*)g_zero_unitsT;
        if (U < HALO_U) lds_dma16(src, s_halo + ub);
    }
    u32x4 wa[WF];
#pragma unroll
    for (int f = 0; f < WF; ++f) wa[f] = wm[((long long)f * 16 + col) * 4 + grp];

    // Wave w: position blocks j < NJ = tile row 2 w + j / BR, columns 16 (j % BR) .. + 15.
    f32x4 acc[MB][NJ];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        f32x4 bv;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int R = 16 * mb + 4 * grp + r, ph = R / COUTP, oc = R % COUTP;
            bv[r] = (ph < 4 && p.bias && oc < p.cout_g) ? p.bias[oc] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[mb][j] = bv;
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's halo loads are in LDS
    __syncthreads();                     // ... and every other wave's
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
#pragma unroll
        for (int n = 0; n < 4; ++n) {
            const int a = n >> 1, b = n & 1, slot = kc * 4 + grp;
            u32x4 bv[NJ];
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const int pix = (2 * wave + j / BR + a) * HX + 16 * (j % BR) + col + b;
                bv[j] = s_halo[pix * SL + (slot ^ swz(pix))];
                if (p.relu6_in) bv[j] = relu6_vec<T>(bv[j]);
            }
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int j = 0; j < NJ; ++j) Mma16<T>::run(acc[mb][j], wa[(kc * 4 + n) * MB + mb], bv[j]);
        }

    // Row R = 16 mb + 4 grp + r of column col: phase R / COUTP, output R % COUTP.
    if constexpr (COUTP == 1) {
        // Only the lanes of K group 0 hold real rows (the four phases of their position). Lane
        // (col, g) takes NJ of them from lane col -- position block jb = g NJ / 4, phases
        // r0 = g NJ % 4 .. r0 + NJ - 1 -- so that every lane stores NJ outputs instead of a
        // quarter of the lanes storing 4 NJ.
        const int jb = (grp * NJ) >> 2, r0 = (grp * NJ) & 3;
        float v[NJ];
#pragma unroll
        for (int k = 0; k < NJ; ++k) v[k] = 0.0f;
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float t = __shfl(acc[0][j][r], col);
#pragma unroll
                for (int k = 0; k < NJ; ++k)
                    if (jb == j && r0 + k == r) v[k] = t;
            }
        const int yq = y0 + 2 * wave + jb / BR, xq = x0 + 16 * (jb % BR) + col;
#pragma unroll
        for (int k = 0; k < NJ; ++k) {
            const int ph = r0 + k;
            const int oy = 2 * yq + (ph >> 1), ox = 2 * xq + (ph & 1);
            if (oy < p.OH && ox < p.OW) epilogue_store<T>(p, bi, oy, ox, 0, 1, f32x4{v[k], 0.0f, 0.0f, 0.0f});
        }
        return;
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int yq = y0 + 2 * wave + j / BR, xq = x0 + 16 * (j % BR) + col;
            if constexpr (COUTP >= 4) {
                // The lane's four rows are four consecutive outputs of one phase.
                const int R0 = 16 * mb + 4 * grp, ph = R0 / COUTP, oc0 = R0 % COUTP;
                const int oy = 2 * yq + (ph >> 1), ox = 2 * xq + (ph & 1);
                if (ph < 4 && oc0 < p.cout_g && oy < p.OH && ox < p.OW)
                    epilogue_store<T>(p, bi, oy, ox, oc0, min(4, p.cout_g - oc0), acc[mb][j]);
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int R = 16 * mb + 4 * grp + r, ph = R / COUTP, oc = R % COUTP;
                    const int oy = 2 * yq + (ph >> 1), ox = 2 * xq + (ph & 1);
                    if (ph < 4 && oc < p.cout_g && oy < p.OH && ox < p.OW)
                        epilogue_store<T>(p, bi, oy, ox, oc, 1, f32x4{acc[mb][j][r], 0.0f, 0.0f, 0.0f});
                }
            }
        }
}

// Whether a layer's tap tables are the 3x3 / padding 1 ones k_convT3_narrow hard-codes
// (halo offsets 1 = input row y', 2 = y' + 1).
static bool taps_are_k3p1(const ConvParams& p) {
    static const int nt[4] = {1, 2, 2, 4};
    static const int dy[4][4] = {{1}, {1, 1}, {2, 1}, {2, 2, 1, 1}};
    static const int dx[4][4] = {{1}, {2, 1}, {1, 1}, {2, 1, 2, 1}};
    for (int ph = 0; ph < 4; ++ph) {
        if (p.ntaps[ph] != nt[ph]) return false;
        for (int t = 0; t < nt[ph]; ++t)
            if (p.tap_dy[ph][t] != dy[ph][t] || p.tap_dx[ph][t] != dx[ph][t]) return false;
    }
    return true;
}

template <typename T>
static hipError_t go_narrow3(int coutp, const ConvParams& p, const float* wn, int cin, hipStream_t s) {
    const int gw = (p.OW + 1) / 2, gh = (p.OH + 1) / 2;
    const long long blocks = ((long long)((gw + 31) / 32) * ((gh + 7) / 8) * p.N + 7) / 8 * 8;
    if (blocks <= 0 || blocks > (1ll << 30) || p.N < 1 || p.N > MAXB) return hipErrorInvalidValue;
    const dim3 g((unsigned)blocks);
    switch (coutp) {
        case 1: hipLaunchKernelGGL((k_convT3_narrow<T, 1>), g, dim3(256), 0, s, p, wn, cin); break;
        case 2: hipLaunchKernelGGL((k_convT3_narrow<T, 2>), g, dim3(256), 0, s, p, wn, cin); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// One or two outputs only: wider layers spend their time in the FMAs, where the generic
// kernel's LDS-broadcast weights beat scalar loads of 9 x coutp weights per input channel.
bool convT_narrow_k3(int dtype, const ConvParams& p, int cin) {
    const int vec = dtype == DT_F32 ? 4 : 8;
    return p.cout_g <= 2 && taps_are_k3p1(p) && cin % (8 * vec) == 0 && p.x.cs % vec == 0 &&
           p.x.c_off % vec == 0 && p.x.row % vec == 0 && p.x.bstride % vec == 0;
}

bool convT_mfma_k3(int dtype, const ConvParams& p, int cin) {
    return dtype != DT_F32 && taps_are_k3p1(p) && (cin == 64 || cin == 128) && p.x.cs % 8 == 0 &&
           p.x.c_off % 8 == 0 && p.x.row % 8 == 0 && p.x.bstride % 8 == 0;
}

template <typename T, int CIN>
static hipError_t go_mfma3(int coutp, const ConvParams& p, const void* wm, hipStream_t s) {
    constexpr int TX = CIN == 128 ? 16 : 32;
    const int gw = (p.OW + 1) / 2, gh = (p.OH + 1) / 2;
    const long long blocks = ((long long)((gw + TX - 1) / TX) * ((gh + 7) / 8) * p.N + 7) / 8 * 8;
    if (blocks <= 0 || blocks > (1ll << 30) || p.N < 1 || p.N > MAXB) return hipErrorInvalidValue;
    const dim3 g((unsigned)blocks);
    const u32x4* w = (const u32x4*)wm;
    switch (coutp) {
        case 1: hipLaunchKernelGGL((k_convT3_mfma<T, 1, CIN, TX>), g, dim3(256), 0, s, p, w); break;
        case 2: hipLaunchKernelGGL((k_convT3_mfma<T, 2, CIN, TX>), g, dim3(256), 0, s, p, w); break;
        case 4: hipLaunchKernelGGL((k_convT3_mfma<T, 4, CIN, TX>), g, dim3(256), 0, s, p, w); break;
        case 8: hipLaunchKernelGGL((k_convT3_mfma<T, 8, CIN, TX>), g, dim3(256), 0, s, p, w); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <typename T>
static hipError_t go_mfma3_c(int coutp, const ConvParams& p, const void* wm, int cin, hipStream_t s) {
    return cin == 128 ? go_mfma3<T, 128>(coutp, p, wm, s) : go_mfma3<T, 64>(coutp, p, wm, s);
}

hipError_t launch_convT3_mfma(int dtype, int coutp, const ConvParams& p, const void* wm, int cin, hipStream_t s) {
    if (!convT_mfma_k3(dtype, p, cin)) return hipErrorInvalidValue;
    switch (dtype) {
        case DT_F16: return go_mfma3_c<_Float16>(coutp, p, wm, cin, s);
        case DT_BF16: return go_mfma3_c<__bf16>(coutp, p, wm, cin, s);
    }
    return hipErrorInvalidValue;
}

template <typename T>
static hipError_t go_narrow(int coutp, const ConvParams& p, const float* wn, int cin, hipStream_t s) {
    const int gw = (p.OW + 1) / 2, gh = (p.OH + 1) / 2;
    const long long blocks = ((long long)((gw + 63) / 64) * ((gh + 3) / 4) * p.N + 7) / 8 * 8;
    if (blocks <= 0 || blocks > (1ll << 30) || p.N < 1 || p.N > MAXB) return hipErrorInvalidValue;
    const dim3 g((unsigned)blocks);
    switch (coutp) {
        case 1: hipLaunchKernelGGL((k_convT_narrow<T, 1>), g, dim3(256), 0, s, p, wn, cin); break;
        case 2: hipLaunchKernelGGL((k_convT_narrow<T, 2>), g, dim3(256), 0, s, p, wn, cin); break;
        case 4: hipLaunchKernelGGL((k_convT_narrow<T, 4>), g, dim3(256), 0, s, p, wn, cin); break;
        case 8: hipLaunchKernelGGL((k_convT_narrow<T, 8>), g, dim3(256), 0, s, p, wn, cin); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_convT_narrow(int dtype, int coutp, const ConvParams& p, const float* wn, int cin,
                               hipStream_t s) {
    if (convT_narrow_k3(dtype, p, cin)) {
        switch (dtype) {
            case DT_F32: return go_narrow3<float>(coutp, p, wn, cin, s);
            case DT_F16: return go_narrow3<_Float16>(coutp, p, wn, cin, s);
            case DT_BF16: return go_narrow3<__bf16>(coutp, p, wn, cin, s);
        }
        return hipErrorInvalidValue;
    }
    switch (dtype) {
        case DT_F32: return go_narrow<float>(coutp, p, wn, cin, s);
        case DT_F16: return go_narrow<_Float16>(coutp, p, wn, cin, s);
        case DT_BF16: return go_narrow<__bf16>(coutp, p, wn, cin, s);
    }
    return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------------------------
// Launch dispatch.
// ---------------------------------------------------------------------------------------------
// The fp32 dense tile shapes run the direct-LDS-load kernel (1x1 layers stage two K chunks per
// barrier); the 16-bit ones and the narrow shapes run conv_igemm.
template <int WC, int WP, int CF, int PF>
constexpr bool use_dma_f32() {
    return (WC == 2 && WP == 2 && CF == 2 && PF == 4) || (WC == 2 && WP == 4 && CF == 2 && PF == 4) ||
           (WC == 4 && WP == 2 && CF == 2 && PF == 4);
}

template <typename T, int KH, int KW, int S, bool TR, int WC, int WP, int CF, int PF>
static hipError_t go(const ConvParams& p0, hipStream_t s) {
    constexpr int SG = (KH * KW == 1 && !TR) ? 4 : 1;
    constexpr int TY = WP * PF;
    ConvParams p = p0;
    const int gh = TR ? (p.OH + 1) / 2 : p.OH;
    const int gw = TR ? (p.OW + 1) / 2 : p.OW;
    if (p.ntiles != p.groups * p.nblk_g / (WC * CF) || p.N < 1 || p.N > MAXB) return hipErrorInvalidValue;
    p.gx = (gw + 15) / 16;
    p.gy = (gh + TY - 1) / TY;
    const long long total = (long long)p.gx * p.gy * p.N * p.ntiles * (TR ? 4 : 1);
    if (total <= 0 || total > (1ll << 30)) return hipErrorInvalidValue;
    if constexpr (sizeof(T) == 4 && use_dma_f32<WC, WP, CF, PF>()) {
        constexpr int SGD = (KH * KW == 1 && !TR) ? 2 : 1;
        hipLaunchKernelGGL((conv_dma_f32<KH, KW, S, TR, WC, WP, CF, PF, SGD>), dim3((unsigned)total),
                           dim3(WC * WP * 64), 0, s, p);
    } else {
        hipLaunchKernelGGL((conv_igemm<T, KH, KW, S, TR, WC, WP, CF, PF, SG>), dim3((unsigned)total),
                           dim3(WC * WP * 64), 0, s, p);
    }
    return hipGetLastError();
}

template <typename T, int WC, int WP, int CF, int PF>
static hipError_t go_kind(int kind, const ConvParams& p, hipStream_t s) {
    switch (kind) {
        case CK_1x1: return go<T, 1, 1, 1, false, WC, WP, CF, PF>(p, s);
        case CK_2x2: return go<T, 2, 2, 1, false, WC, WP, CF, PF>(p, s);
        case CK_3x3: return go<T, 3, 3, 1, false, WC, WP, CF, PF>(p, s);
        case CK_3x3_S2: return go<T, 3, 3, 2, false, WC, WP, CF, PF>(p, s);
        case CK_T3: return go<T, 3, 3, 1, true, WC, WP, CF, PF>(p, s);
    }
    return hipErrorInvalidValue;
}

// Instantiated tile shapes: (wc, wp, cf, pf).
//   {2,2,2,4}: 64 channels x 8 rows, 4 waves  (dense layers)
//   {2,4,2,4}: 64 channels x 16 rows, 8 waves (dense stride-1 3x3 layers only)
//   {4,2,2,4}: 128 channels x 8 rows, 8 waves (fp32 1x1 layers with >= 256 outputs only)
//   {1,4,2,2}: 32 channels x 8 rows  (32-channel groups / outputs)
//   {1,4,1,2}: 16 channels x 8 rows  (16-channel groups / narrow outputs)
#define ZJAI_CFGS(X) X(2, 2, 2, 4) X(1, 4, 2, 2) X(1, 4, 1, 2)

template <typename T>
static hipError_t go_cfg(int kind, TileCfg c, const ConvParams& p, hipStream_t s) {
    if (c.wc == 2 && c.wp == 4 && c.cf == 2 && c.pf == 4)
        return kind == CK_3x3 ? go<T, 3, 3, 1, false, 2, 4, 2, 4>(p, s) : hipErrorInvalidValue;
    if (c.wc == 4 && c.wp == 2 && c.cf == 2 && c.pf == 4) {
        if constexpr (sizeof(T) == 4) return kind == CK_1x1 ? go<T, 1, 1, 1, false, 4, 2, 2, 4>(p, s) : hipErrorInvalidValue;
        return kind == CK_3x3_S2 ? go<T, 3, 3, 2, false, 4, 2, 2, 4>(p, s) : hipErrorInvalidValue;
    }
#define ZJAI_GO(a, b, cc, d) \
    if (c.wc == a && c.wp == b && c.cf == cc && c.pf == d) return go_kind<T, a, b, cc, d>(kind, p, s);
    ZJAI_CFGS(ZJAI_GO)
#undef ZJAI_GO
    return hipErrorInvalidValue;
}

hipError_t launch_conv(int kind, int dtype, TileCfg cfg, const ConvParams& p, hipStream_t s) {
    switch (dtype) {
        case DT_F32: return go_cfg<float>(kind, cfg, p, s);
        case DT_F16: return go_cfg<_Float16>(kind, cfg, p, s);
        case DT_BF16: return go_cfg<__bf16>(kind, cfg, p, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace zjai
