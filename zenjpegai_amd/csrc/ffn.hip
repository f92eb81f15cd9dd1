// The feed-forward half of a transformer block as one kernel (16-bit storage types here; the f32
// form, k_ffn_f32, follows the same plan with the LayerNorm output in registers):
//   u = LayerNorm(x); p = project_in(u) (1x1, dim -> 2 * hid); d = depthwise3x3(p);
//   g = elu(d[:hid]) * d[hid:]; y = x + project_out(g) (1x1, hid -> dim)
// (TransformerBlock::forward, src/model/attention.rs:346-369; LayerNorm :267-279).
//
// Unfused, the 2 * hid = 8 * dim channel tensor p and the hid-channel g make the round trip to
// HBM (6.8 KB per position at dim 128 in bf16, against 0.5 KB for x and y); here they never
// leave the workgroup. One workgroup (8 waves) owns a 14 x 14 output tile and its 16 x 16 halo
// (256 positions):
//   1. loads x over the halo, LayerNorms every halo position into LDS (u, storage type);
//   2. for each slice of 32 gate pairs (p channels j and hid + j, j in [32 s, 32 s + 32)):
//      a. p slice [256 positions x 64 channels] = u x W_in slice on v_mfma_f32_16x16x32
//         (bias first, then K in 32-channel chunks: the unfused 1x1 conv's instruction
//         sequence), rounded to the storage type, zero outside the picture (the depthwise
//         conv's zero padding) -> LDS;
//      b. depthwise 3x3 + ELU gate on the 14 x 14 interior (f32 FMAs in the unfused kernel's
//         order), rounded to the storage type -> LDS;
//      c. y accumulators [dim x 196] += W_out slice x g slice on v_mfma_f32_16x16x32 (the
//         slice is the packed project_out weight's K chunk s, so K runs in channel order).
//   3. adds the residual x and stores y through an LDS transpose (whole channel runs per
//      position).
// Every intermediate is rounded to the storage type exactly where the unfused path stores it
// and every sum runs in the unfused kernels' order, so the two paths agree bit for bit.
// The weights of slice s + 1 are fetched into registers while slice s computes.

#include "mfma.h"
#include "ops.h"

namespace zjai {

namespace {

__device__ u32x4 g_zero16[1];  // 16 zero bytes: the source of absent biases

constexpr int FT = 14;          // output tile side
constexpr int FH = FT + 2;      // halo side
constexpr int FNP = FH * FH;    // halo positions (256: sixteen 16-position MFMA blocks)
constexpr int FOP = FT * FT;    // output positions (196)
constexpr int FPB = 13;         // 16-position blocks covering the output positions
constexpr int FTHREADS = 512;

template <typename T>
__device__ __forceinline__ void unpack8(u32x4 v, float (&o)[8]) {
    typedef T t8 __attribute__((ext_vector_type(8)));
    const t8 hv = __builtin_bit_cast(t8, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = (float)hv[i];
}

template <typename T>
__device__ __forceinline__ u32x4 pack8(const float (&f)[8]) {
    typedef T t8 __attribute__((ext_vector_type(8)));
    t8 hv;
#pragma unroll
    for (int i = 0; i < 8; ++i) hv[i] = (T)f[i];
    return __builtin_bit_cast(u32x4, hv);
}

template <typename T>
__device__ __forceinline__ void unpack2(unsigned v, float (&o)[2]) {
    typedef T t2 __attribute__((ext_vector_type(2)));
    const t2 hv = __builtin_bit_cast(t2, v);
    o[0] = (float)hv[0];
    o[1] = (float)hv[1];
}

// Unit swizzle of a p-slice row in k_ffn (a position's 64 channels = 8 16-byte units; unit q
// sits at q ^ pswz(column), column = position % 16). gfx950 serves a ds_read_b32 in two passes
// of 32 lanes over 32 banks (128 bytes): the 32 lanes of a pass are two neighbouring columns'
// 16 lanes, each reading 64 bytes (one half) of its 128-byte row, so bit 2 of the swizzle -- the
// half the column's 64 bytes land in -- is the column's parity. Over 16 columns the swizzle
// takes every value twice: the project_in stores (ds_write_b64, 16 lanes per pass) stay at the
// two passes a fixed 8-byte half needs.
__device__ __forceinline__ int pswz(int c) { return ((c & 1) << 2) | ((c >> 1) & 3); }

// Unit swizzle of the rows of 4 16-byte units that one 16x16x32 fragment read takes 16 of
// (g and W_out in k_ffn): unit q of row r at q ^ gswz(r). A ds_read_b128 runs in four passes of
// 16 lanes (lane l in pass (l / 32, parity of bits 2..4 of l)) over 64 banks; flipping bit 1
// of the unit in rows with bit 2 set puts each pass's 16 rows on distinct bank quads.
__device__ __forceinline__ int gswz(int r) { return (r & 4) >> 1; }

// u rows (halo positions, DIM channels of the storage type, UPR = DIM / 8 16-byte units): unit
// q of row r sits at q ^ ukey(r), so that the 16 rows one half-wave reads for an MFMA fragment
// cover all 16 four-bank groups.
template <int DIM>
__device__ __forceinline__ int ukey(int r) {
    constexpr int UPR = DIM / 8, KSH = DIM == 128 ? 0 : 1;
    return (r >> KSH) & (UPR - 1);
}

// x over the 16 x 16 halo of the tile at (y0, x0) (zero outside the picture) -> LayerNorm per
// position, in place, into s_u (storage type, swizzled rows), as k_layer_norm computes it: f64
// sums in channel order, mean and sqrt(var / C + 1e-5) narrowed to f32, then
// ((x - m) / d) * w + b per element. s_stat: 2 x FNP floats. Ends without a barrier.
template <typename T, int DIM>
__device__ __forceinline__ void ln_halo(const T* xb, const View& xv, int y0, int x0, int h, int w,
                                        const float* ln_w, const float* ln_b, u32x4* s_u,
                                        float* s_stat, int tid) {
    constexpr int UPR = DIM / 8, LN_PT = FNP * UPR / FTHREADS;
    static_assert((FNP * UPR) % FTHREADS == 0, "halo shape");
    // Every load is issued before the first is used: each reads the clamped (in-picture) pixel
    // and positions outside the picture take zeros afterwards, so no load sits in a branch that
    // would wait for it before the next one issues.
    u32x4 xv8[LN_PT];
    bool in8[LN_PT];
#pragma unroll
    for (int i = 0; i < LN_PT; ++i) {
        const int u = tid + i * FTHREADS, pos = u / UPR, q = u % UPR;
        const int iy = y0 - 1 + pos / FH, ix = x0 - 1 + pos % FH;
        in8[i] = iy >= 0 && iy < h && ix >= 0 && ix < w;
        const int cy = min(max(iy, 0), h - 1), cx = min(max(ix, 0), w - 1);
        xv8[i] = *(const u32x4*)(xb + (long long)cy * xv.row + (long long)cx * xv.cs + q * 8);
    }
#pragma unroll
    for (int i = 0; i < LN_PT; ++i) {
        const int u = tid + i * FTHREADS, pos = u / UPR, q = u % UPR;
        s_u[pos * UPR + (q ^ ukey<DIM>(pos))] = in8[i] ? xv8[i] : u32x4{0u, 0u, 0u, 0u};
    }
    __syncthreads();
    if (tid < FNP) {
        const int pos = tid;
        double mean = 0.0;
#pragma unroll 2
        for (int q = 0; q < UPR; ++q) {
            float f[8];
            unpack8<T>(s_u[pos * UPR + (q ^ ukey<DIM>(pos))], f);
#pragma unroll
            for (int k = 0; k < 8; ++k) mean += (double)f[k];
        }
        mean /= (double)DIM;
        double var = 0.0;
#pragma unroll 2
        for (int q = 0; q < UPR; ++q) {
            float f[8];
            unpack8<T>(s_u[pos * UPR + (q ^ ukey<DIM>(pos))], f);
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const double e = (double)f[k] - mean;
                var = var + e * e;
            }
        }
        s_stat[pos] = (float)mean;
        s_stat[FNP + pos] = sqrtf((float)(var / (double)DIM) + 1e-5f);
    }
    __syncthreads();
    const int q = tid % UPR;  // the same unit for every i (FTHREADS % UPR == 0)
    float lw[8], lb[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        lw[k] = ln_w[q * 8 + k];
        lb[k] = ln_b[q * 8 + k];
    }
#pragma unroll 2
    for (int i = 0; i < LN_PT; ++i) {
        const int pos = (tid + i * FTHREADS) / UPR;
        u32x4* a = &s_u[pos * UPR + (q ^ ukey<DIM>(pos))];
        float f[8];
        unpack8<T>(*a, f);
        const float m = s_stat[pos], d = s_stat[FNP + pos];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            float e = f[k] - m;
            e = e / d;
            e = e * lw[k];
            f[k] = e + lb[k];
        }
        *a = pack8<T>(f);
    }
}

}  // namespace

template <typename T, int DIM>
__global__ void __launch_bounds__(FTHREADS) k_ffn(const FfnArgs p) {
    constexpr int HID = 4 * DIM, C2 = 2 * HID, NS = HID / 32;
    constexpr int UPR = DIM / 8;  // 16-byte units per u / W_in row
    // u and W_in rows are swizzled by ukey (16-byte unit q of row r at q ^ ukey(r)).
    constexpr int CB2 = DIM / 16, WPC = 8 / CB2, NPB = (FPB + WPC - 1) / WPC;
    constexpr int U_U = FNP * UPR, WIN_U = 64 * UPR, P_U = FNP * 8, G_U = FPB * 16 * 4, WO_U = DIM * 4;
    constexpr int WIN_PT = WIN_U / FTHREADS;
    static_assert(WIN_U % FTHREADS == 0 && U_U % FTHREADS == 0 && WO_U <= FTHREADS, "fetch shapes");
    static_assert(FOP * (DIM + 4) * 4 <= (U_U + WIN_U + P_U) * 16, "output transpose fits");
    // Per slice also b_in [64] and the depthwise weights [9][64] + bias [64] (f32), two buffers.
    constexpr int BIN_U = 16, DWW_U = (9 * 64 + 64) / 4, X_U = BIN_U + DWW_U;
    static_assert(X_U <= FTHREADS, "fetch shapes");
    __shared__ u32x4 s_lds[U_U + WIN_U + P_U + G_U + 2 * WO_U + 2 * X_U];
    __shared__ float s_stat[2 * FNP];
    u32x4* s_u = s_lds;
    u32x4* s_win = s_u + U_U;
    u32x4* s_p = s_win + WIN_U;
    u32x4* s_g = s_p + P_U;
    u32x4* s_wo = s_g + G_U;
    u32x4* s_x = s_wo + 2 * WO_U;  // [2][b_in 16 units, depthwise 160 units]
    auto key = [](int r) { return ukey<DIM>(r); };

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, grp = lane >> 4;  // 16x16 MFMA fragment lane
    const int bid = (int)blockIdx.x;
    const int tx = bid % p.gx, ty = (bid / p.gx) % p.gy, b = bid / (p.gx * p.gy);
    const int y0 = ty * FT, x0 = tx * FT;
    const T* xb = (const T*)p.x.p + (long long)b * p.x.bstride + p.x.c_off;
    const T* w_in = (const T*)p.w_in;
    const T* w_out = (const T*)p.w_out;

    // Slice s weights: W_in rows j and hid + j (j in [32 s, 32 s + 32)) of the packed 1x1
    // weight [chunk][nblk][16][32]; W_out = chunk s of the packed project_out weight.
    u32x4 rwi[WIN_PT], rwo = {0u, 0u, 0u, 0u}, rx = {0u, 0u, 0u, 0u};
    auto gch = [](int s, int l) { return l < 32 ? 32 * s + l : HID + 32 * s + (l - 32); };
    auto fetch_w = [&](int s) {
#pragma unroll
        for (int i = 0; i < WIN_PT; ++i) {
            const int u = tid + i * FTHREADS, r = u / UPR, q = u % UPR;
            const int o = r < 32 ? 32 * s + r : HID + 32 * s + (r - 32);
            const long long off = ((long long)((q >> 2) * p.nblk_in + (o >> 4)) * 16 + (o & 15)) * 32 + (q & 3) * 8;
            rwi[i] = *(const u32x4*)(w_in + off);
        }
        if (tid < WO_U) {
            const int r = tid >> 2, q = tid & 3;
            const long long off = ((long long)(s * p.nblk_out + (r >> 4)) * 16 + (r & 15)) * 32 + q * 8;
            rwo = *(const u32x4*)(w_out + off);
        }
        // Thread u < 16: b_in of local channels 4u..4u+3; 16 <= u < 160: depthwise tap
        // (u - 16) / 16 of local channels 4 (u % 16)..; 160 <= u < 176: depthwise bias; absent
        // biases and threads >= 176 read zeros. One load per thread at a selected address, so
        // nothing waits for it before its use in put_w.
        const float* src = reinterpret_cast<const float*>(g_zero16);
        if (tid < BIN_U) {
            if (p.b_in) src = p.b_in + gch(s, 4 * tid);
        } else if (tid < BIN_U + 144) {
            const int u = tid - BIN_U;
            src = p.dw_w + (u >> 4) * C2 + gch(s, 4 * (u & 15));
        } else if (tid < X_U && p.dw_b) {
            src = p.dw_b + gch(s, 4 * (tid - BIN_U - 144));
        }
        rx = *(const u32x4*)src;
    };
    auto put_w = [&](int s) {
#pragma unroll
        for (int i = 0; i < WIN_PT; ++i) {
            const int u = tid + i * FTHREADS, r = u / UPR, q = u % UPR;
            s_win[r * UPR + (q ^ key(r))] = rwi[i];
        }
        if (tid < WO_U) s_wo[(s & 1) * WO_U + (tid & ~3) + ((tid & 3) ^ gswz(tid >> 2))] = rwo;
        if (tid < X_U) s_x[(s & 1) * X_U + tid] = rx;
    };

    // ---- 1. x over the halo (zero outside the picture), then LayerNorm in place.
    fetch_w(0);
    ln_halo<T, DIM>(xb, p.x, y0, x0, p.h, p.w, p.ln_w, p.ln_b, s_u, s_stat, tid);
    put_w(0);

    // ---- 2. slices of 32 gate pairs.
    const int cb1 = wave & 1;            // GEMM1 half (0: first-half channels, 1: second half)
    const int pb1 = wave >> 1;           // GEMM1 position blocks 4 pb1 .. 4 pb1 + 3
    const int cb2 = wave % CB2;          // GEMM2 output-channel block
    const int pw2 = wave / CB2;          // GEMM2 position blocks pw2 + WPC * i
    f32x4 acc2[NPB];
    {
        f32x4 bo;
#pragma unroll
        for (int r = 0; r < 4; ++r) bo[r] = p.b_out ? p.b_out[cb2 * 16 + 4 * grp + r] : 0.0f;
#pragma unroll
        for (int i = 0; i < NPB; ++i) acc2[i] = bo;
    }
    // Depthwise role: thread (pair group pg, column c, row half rh) for tid < 28 * 16.
    const int pg = tid & 15, dc = (tid >> 4) % FT, rh = (tid >> 4) / FT;
    const bool dw_thread = tid < 2 * FT * 16;

    // Phase a of slice s: p slice = bias + u x W_in into LDS.
    auto phase_a = [&](int s) __attribute__((always_inline)) {
        // a. p slice = bias + u x W_in: the two 16-channel blocks of half cb1 (0: channels
        //    32 s .., 1: hid + 32 s ..) x position blocks 4 pb1 .. 4 pb1 + 3.
        //    16x16x32 MFMAs with K in 32-channel chunks, bias first: the unfused 1x1 conv's
        //    instruction sequence, so p matches it bit for bit.
        f32x4 acc1[2][4];
        const float* sbin = reinterpret_cast<const float*>(s_x + (s & 1) * X_U);
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            f32x4 bi;
#pragma unroll
            for (int r = 0; r < 4; ++r) bi[r] = sbin[cb1 * 32 + c * 16 + 4 * grp + r];
#pragma unroll
            for (int i = 0; i < 4; ++i) acc1[c][i] = bi;
        }
#pragma unroll
        for (int kc = 0; kc < DIM / 32; ++kc) {
            const int q = 4 * kc + grp;
            u32x4 a[2], bv[4];
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const int ra = cb1 * 32 + c * 16 + col;
                a[c] = s_win[ra * UPR + (q ^ key(ra))];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int rb = (pb1 * 4 + i) * 16 + col;
                bv[i] = s_u[rb * UPR + (q ^ key(rb))];
            }
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int i = 0; i < 4; ++i) Mma16<T>::run(acc1[c][i], a[c], bv[i]);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int pos = (pb1 * 4 + i) * 16 + col;
            const int iy = y0 - 1 + pos / FH, ix = x0 - 1 + pos % FH;
            const bool inside = iy >= 0 && iy < p.h && ix >= 0 && ix < p.w;
            const int sw = pswz(pos & (FH - 1));  // unit swizzle of the position's row (see the dw reads)
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                typedef T t4 __attribute__((ext_vector_type(4)));
                t4 v;
#pragma unroll
                for (int k = 0; k < 4; ++k) v[k] = inside ? (T)acc1[c][i][k] : (T)0.0f;
                const int ch = cb1 * 32 + c * 16 + 4 * grp;  // local channel (0..63)
                T* dst = (T*)s_p + pos * 64 + ((ch >> 3) ^ sw) * 8 + (ch & 7);
                *reinterpret_cast<t4*>(dst) = v;
            }
        }
    };
    // Phase b of slice s: depthwise 3x3 + gate, p -> g.
    auto phase_b = [&](int s) __attribute__((always_inline)) {
        // b. depthwise 3x3 + gate: rows 7 rh .. 7 rh + 6 of column dc, pairs 32 s + 2 pg + {0, 1}.
        if (dw_thread) {
            // Local channel 2 pg + k (first half) and 32 + 2 pg + k (second half).
            const float* dww = reinterpret_cast<const float*>(s_x + (s & 1) * X_U + BIN_U);
            float wa[9][2], wb[9][2], ba[2], bb[2];
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                ba[k] = dww[576 + 2 * pg + k];
                bb[k] = dww[576 + 32 + 2 * pg + k];
#pragma unroll
                for (int tp = 0; tp < 9; ++tp) {
                    wa[tp][k] = dww[tp * 64 + 2 * pg + k];
                    wb[tp][k] = dww[tp * 64 + 32 + 2 * pg + k];
                }
            }
            // 16-byte unit (pg / 4) of the first half, 4 + pg / 4 of the second, each XORed with
            // pswz(column): the 16 lanes of a position read four units of its row, and the two
            // neighbouring positions of one read pass sit on disjoint banks. The swizzle of halo
            // position (hr, dc + kx) depends on its column dc + kx only (FH = 16), so each read is
            // a per-kx offset plus hr rows.
            static_assert(FH == 16, "row swizzle");
            int offa[3], offb[3];
#pragma unroll
            for (int kx = 0; kx < 3; ++kx) {
                const int c = dc + kx, sw = pswz(c);
                offa[kx] = c * 64 + 2 * (pg & 3) + ((pg >> 2) ^ sw) * 8;
                offb[kx] = c * 64 + 2 * (pg & 3) + ((4 + (pg >> 2)) ^ sw) * 8;
            }
            auto ld = [&](int hr, int kx, float (&oa)[2], float (&ob)[2]) {
                const T* rows = (const T*)s_p + hr * (FH * 64);
                unpack2<T>(*(const unsigned*)(rows + offa[kx]), oa);
                unpack2<T>(*(const unsigned*)(rows + offb[kx]), ob);
            };
            float xa[3][3][2], xb[3][3][2];
            const int r0 = rh * (FT / 2);
#pragma unroll
            for (int kx = 0; kx < 3; ++kx) {
                ld(r0, kx, xa[0][kx], xb[0][kx]);
                ld(r0 + 1, kx, xa[1][kx], xb[1][kx]);
            }
#pragma unroll
            for (int r = 0; r < FT / 2; ++r) {
                const int oy = r0 + r;
#pragma unroll
                for (int kx = 0; kx < 3; ++kx) ld(oy + 2, kx, xa[2][kx], xb[2][kx]);
                float g[2];
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    float a = ba[k], bq = bb[k];
#pragma unroll
                    for (int ky = 0; ky < 3; ++ky)
#pragma unroll
                        for (int kx = 0; kx < 3; ++kx) {
                            a = fmaf(wa[ky * 3 + kx][k], xa[ky][kx][k], a);
                            bq = fmaf(wb[ky * 3 + kx][k], xb[ky][kx][k], bq);
                        }
                    g[k] = elu_fast16(a) * bq;
                }
                typedef T t2 __attribute__((ext_vector_type(2)));
                const int gp = oy * FT + dc;  // g row; its unit pg / 4 swizzled by gswz
                *reinterpret_cast<t2*>((T*)s_g + gp * 32 + ((pg >> 2) ^ gswz(gp)) * 8 + 2 * (pg & 3)) =
                    t2{(T)g[0], (T)g[1]};
#pragma unroll
                for (int kx = 0; kx < 3; ++kx)
#pragma unroll
                    for (int k = 0; k < 2; ++k) {
                        xa[0][kx][k] = xa[1][kx][k];
                        xa[1][kx][k] = xa[2][kx][k];
                        xb[0][kx][k] = xb[1][kx][k];
                        xb[1][kx][k] = xb[2][kx][k];
                    }
            }
        }
    };
    // Phase c of slice s: y += W_out(s) x g.
    auto phase_c = [&](int s) __attribute__((always_inline)) {
        // c. y += W_out(s) x g (output-channel block cb2, position blocks pw2 + WPC * i).
        const u32x4 a = s_wo[(s & 1) * WO_U + (cb2 * 16 + col) * 4 + (grp ^ gswz(col))];
#pragma unroll
        for (int i = 0; i < NPB; ++i) {
            const int pb = pw2 + WPC * i;
            if (pb < FPB) Mma16<T>::run(acc2[i], a, s_g[(pb * 16 + col) * 4 + (grp ^ gswz(col))]);
        }
    };

    // Two barriers per slice: phase c of slice s and phase a of slice s + 1 share one barrier
    // interval (c reads g and W_out(s); a reads u, W_in(s + 1) and writes p, which every wave
    // finished reading before the barrier ahead of c). Per accumulator the MFMAs run in the same
    // order as with a barrier between them.
    __syncthreads();  // u, W_in(0), W_out(0) ready
    if (NS > 1) fetch_w(1);
    phase_a(0);
    for (int s = 0; s < NS; ++s) {
        __syncthreads();  // p(s) ready; W_in(s) consumed; g and W_out(s - 1) free
        if (s + 1 < NS) put_w(s + 1);
        phase_b(s);
        __syncthreads();  // g(s) ready; W(s + 1) in LDS; p free
        if (s + 2 < NS) fetch_w(s + 2);
        phase_c(s);
        if (s + 1 < NS) phase_a(s + 1);
    }

    // ---- 3. y = acc + x through an LDS transpose.
    __syncthreads();
    constexpr int OLD = DIM + 4;
    float* so = reinterpret_cast<float*>(s_lds);
#pragma unroll
    for (int i = 0; i < NPB; ++i) {
        const int pb = pw2 + WPC * i, pos = pb * 16 + col;
        if (pb < FPB && pos < FOP) {
            float* d = so + pos * OLD + cb2 * 16 + 4 * grp;
#pragma unroll
            for (int r = 0; r < 4; ++r) d[r] = acc2[i][r];
        }
    }
    __syncthreads();
    // 16-byte units (8 channels) of the 196 output positions: every thread issues all of its
    // residual loads before the first add, so their latencies overlap instead of adding up.
    T* yb = (T*)p.y.p + (long long)b * p.y.bstride + p.y.c_off;
    constexpr int U8 = DIM / 8, NU = FOP * U8, EIT = (NU + FTHREADS - 1) / FTHREADS, EG = 4;
#pragma unroll
    for (int i0 = 0; i0 < EIT; i0 += EG) {
        u32x4 rres[EG];
#pragma unroll
        for (int j = 0; j < EG; ++j) {
            const int u = tid + (i0 + j) * FTHREADS, pos = u / U8, q = u % U8;
            const int oy = min(y0 + pos / FT, p.h - 1), ox = min(x0 + pos % FT, p.w - 1);
            rres[j] = u32x4{0u, 0u, 0u, 0u};
            if (i0 + j < EIT && u < NU)  // (clamped pixel: loads issue back to back; unused beyond the picture)
                rres[j] = *(const u32x4*)(xb + (long long)oy * p.x.row + (long long)ox * p.x.cs + q * 8);
        }
#pragma unroll
        for (int j = 0; j < EG; ++j) {
            const int u = tid + (i0 + j) * FTHREADS, pos = u / U8, q = u % U8;
            const int oy = y0 + pos / FT, ox = x0 + pos % FT;
            if (i0 + j >= EIT || u >= NU || oy >= p.h || ox >= p.w) continue;
            const float* sv = so + pos * OLD + q * 8;
            float r[8], v[8];
            unpack8<T>(rres[j], r);
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = sv[k] + r[k];
            *(u32x4*)(yb + (long long)oy * p.y.row + (long long)ox * p.y.cs + q * 8) = pack8<T>(v);
        }
    }
}

// The first half of a transformer block's attention branch as one kernel (16-bit storage
// types): qkv = depthwise3x3(conv1x1(LayerNorm(x))), dim -> 3 dim channels
// (TransformerBlock::forward, src/model/attention.rs:330-333: `prep_data`). Per 14 x 14 tile
// (16 x 16 halo, 8 waves): the LayerNorm prologue of k_ffn, then per slice of 64 of the 3 dim
// channels the 1x1 on 16x16x32 MFMAs (the unfused conv's instruction sequence) into LDS, zero
// outside the picture, and the depthwise 3x3 in the unfused kernel's FMA order, stored to qkv.
// The LayerNorm output and the 1x1's output never reach HBM; the results equal the unfused
// kernels' bit for bit.
template <typename T, int DIM>
__global__ void __launch_bounds__(FTHREADS) k_qkv(const QkvArgs p) {
    constexpr int C3 = 3 * DIM, NS = C3 / 64, UPR = DIM / 8;
    constexpr int U_U = FNP * UPR, WIN_U = 64 * UPR, P_U = FNP * 8;
    // Per slice: conv1 bias [64], depthwise weights [9][64] and bias [64] (f32), two buffers.
    constexpr int BIN_U = 16, X_U = (64 + 9 * 64 + 64) / 4;
    constexpr int WIN_PT = WIN_U / FTHREADS;
    static_assert(WIN_U % FTHREADS == 0 && X_U <= FTHREADS && C3 % 64 == 0, "fetch shapes");
    __shared__ u32x4 s_lds[U_U + WIN_U + P_U + 2 * X_U];
    __shared__ float s_stat[2 * FNP];
    u32x4* s_u = s_lds;
    u32x4* s_win = s_u + U_U;
    u32x4* s_p = s_win + WIN_U;
    u32x4* s_x = s_p + P_U;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, grp = lane >> 4;  // 16x16 MFMA fragment lane
    const int bid = (int)blockIdx.x;
    const int tx = bid % p.gx, ty = (bid / p.gx) % p.gy, b = bid / (p.gx * p.gy);
    const int y0 = ty * FT, x0 = tx * FT;
    const T* xb = (const T*)p.x.p + (long long)b * p.x.bstride + p.x.c_off;
    const T* w1 = (const T*)p.w1;

    // Slice s: conv1 output channels 64 s .. 64 s + 63 (rows of the packed 1x1 weight
    // [chunk][nblk][16][32]), their biases, depthwise taps and depthwise biases.
    u32x4 rwi[WIN_PT], rx = {0u, 0u, 0u, 0u};
    auto fetch = [&](int s) {
#pragma unroll
        for (int i = 0; i < WIN_PT; ++i) {
            const int u = tid + i * FTHREADS, r = u / UPR, q = u % UPR, o = 64 * s + r;
            const long long off = ((long long)((q >> 2) * p.nblk1 + (o >> 4)) * 16 + (o & 15)) * 32 + (q & 3) * 8;
            rwi[i] = *(const u32x4*)(w1 + off);
        }
        // One load per thread at a selected address (zeros for absent biases and threads
        // >= X_U), so nothing waits for it before its use in put.
        const float* src = reinterpret_cast<const float*>(g_zero16);
        if (tid < BIN_U) {
            if (p.b1) src = p.b1 + 64 * s + 4 * tid;
        } else if (tid < BIN_U + 144) {
            const int u = tid - BIN_U;
            src = p.dw_w + (u >> 4) * C3 + 64 * s + 4 * (u & 15);
        } else if (tid < X_U && p.dw_b) {
            src = p.dw_b + 64 * s + 4 * (tid - BIN_U - 144);
        }
        rx = *(const u32x4*)src;
    };
    auto put = [&](int s) {
#pragma unroll
        for (int i = 0; i < WIN_PT; ++i) {
            const int u = tid + i * FTHREADS, r = u / UPR, q = u % UPR;
            s_win[r * UPR + (q ^ ukey<DIM>(r))] = rwi[i];
        }
        if (tid < X_U) s_x[(s & 1) * X_U + tid] = rx;
    };

    fetch(0);
    ln_halo<T, DIM>(xb, p.x, y0, x0, p.h, p.w, p.ln_w, p.ln_b, s_u, s_stat, tid);
    put(0);

    const int cb1 = wave & 1;   // conv1 channel blocks 2 cb1, 2 cb1 + 1 of the slice
    const int pb1 = wave >> 1;  // conv1 position blocks 4 pb1 .. 4 pb1 + 3
    // Depthwise role (tid < 448, whole waves 0-6): channel pair pg, column dc, all 14 rows.
    const int pg = tid & 31, dc = (tid >> 5) % FT;
    const bool dw_thread = tid < 32 * FT;
    T* yb = (T*)p.y.p + (long long)b * p.y.bstride + p.y.c_off;

    for (int s = 0; s < NS; ++s) {
        __syncthreads();  // u, W1(s) ready; p free
        if (s + 1 < NS) fetch(s + 1);
        const float* sx = reinterpret_cast<const float*>(s_x + (s & 1) * X_U);
        {
            f32x4 acc1[2][4];
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                f32x4 bi;
#pragma unroll
                for (int r = 0; r < 4; ++r) bi[r] = sx[cb1 * 32 + c * 16 + 4 * grp + r];
#pragma unroll
                for (int i = 0; i < 4; ++i) acc1[c][i] = bi;
            }
#pragma unroll
            for (int kc = 0; kc < DIM / 32; ++kc) {
                const int q = 4 * kc + grp;
                u32x4 a[2], bv[4];
#pragma unroll
                for (int c = 0; c < 2; ++c) {
                    const int ra = cb1 * 32 + c * 16 + col;
                    a[c] = s_win[ra * UPR + (q ^ ukey<DIM>(ra))];
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int rb = (pb1 * 4 + i) * 16 + col;
                    bv[i] = s_u[rb * UPR + (q ^ ukey<DIM>(rb))];
                }
#pragma unroll
                for (int c = 0; c < 2; ++c)
#pragma unroll
                    for (int i = 0; i < 4; ++i) Mma16<T>::run(acc1[c][i], a[c], bv[i]);
            }
            T* sp = reinterpret_cast<T*>(s_p);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int pos = (pb1 * 4 + i) * 16 + col;
                const int iy = y0 - 1 + pos / FH, ix = x0 - 1 + pos % FH;
                const bool inside = iy >= 0 && iy < p.h && ix >= 0 && ix < p.w;
#pragma unroll
                for (int c = 0; c < 2; ++c) {
                    typedef T t4 __attribute__((ext_vector_type(4)));
                    t4 v;
#pragma unroll
                    for (int k = 0; k < 4; ++k) v[k] = inside ? (T)acc1[c][i][k] : (T)0.0f;
                    // 16-byte units of a position's row XORed with pos & 7: the 16 positions of
                    // one store spread over all banks (the depthwise reads use the same map).
                    const int ch = cb1 * 32 + c * 16 + 4 * grp;
                    *reinterpret_cast<t4*>(sp + pos * 64 + ((ch >> 3) ^ (pos & 7)) * 8 + (ch & 7)) = v;
                }
            }
        }
        __syncthreads();  // p ready; W1(s) consumed
        if (s + 1 < NS) put(s + 1);
        if (dw_thread) {
            // Channels 2 pg, 2 pg + 1 of the slice; acc = bias, then (ky, kx) ascending.
            const float* dww = sx + BIN_U * 4;
            float wv[9][2], bv[2];
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                bv[k] = dww[576 + 2 * pg + k];
#pragma unroll
                for (int tp = 0; tp < 9; ++tp) wv[tp][k] = dww[tp * 64 + 2 * pg + k];
            }
            const T* sp = reinterpret_cast<const T*>(s_p) + 2 * (pg & 3);
            float xw[3][3][2];
            // The swizzle pos & 7 of halo position (hr, dc + kx) is (dc + kx) & 7 (FH is a
            // multiple of 8), so each read is a per-kx offset plus hr rows.
            static_assert(FH % 8 == 0, "row swizzle");
            int off[3];
#pragma unroll
            for (int kx = 0; kx < 3; ++kx) off[kx] = (dc + kx) * 64 + ((pg >> 2) ^ ((dc + kx) & 7)) * 8;
            auto ld = [&](int hr, int kx, float (&o)[2]) {
                unpack2<T>(*(const unsigned*)(sp + hr * (FH * 64) + off[kx]), o);
            };
#pragma unroll
            for (int kx = 0; kx < 3; ++kx) {
                ld(0, kx, xw[0][kx]);
                ld(1, kx, xw[1][kx]);
            }
            const int ox = x0 + dc;
#pragma unroll
            for (int r = 0; r < FT; ++r) {
#pragma unroll
                for (int kx = 0; kx < 3; ++kx) ld(r + 2, kx, xw[2][kx]);
                float o[2];
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    float a = bv[k];
#pragma unroll
                    for (int ky = 0; ky < 3; ++ky)
#pragma unroll
                        for (int kx = 0; kx < 3; ++kx) a = fmaf(wv[ky * 3 + kx][k], xw[ky][kx][k], a);
                    o[k] = a;
                }
                const int oy = y0 + r;
                if (oy < p.h && ox < p.w) {
                    typedef T t2 __attribute__((ext_vector_type(2)));
                    *reinterpret_cast<t2*>(yb + (long long)oy * p.y.row + (long long)ox * p.y.cs + 64 * s + 2 * pg) =
                        t2{(T)o[0], (T)o[1]};
                }
#pragma unroll
                for (int kx = 0; kx < 3; ++kx)
#pragma unroll
                    for (int k = 0; k < 2; ++k) {
                        xw[0][kx][k] = xw[1][kx][k];
                        xw[1][kx][k] = xw[2][kx][k];
                    }
            }
        }
    }
}

// ------------------------------------------------------------------------- f32 storage
// The same two kernels for f32 nets. A 16 x 16 halo of f32 LayerNorm output (128 KB at dim 128)
// does not fit LDS beside the slice buffers, so each wave keeps the LayerNorm output of its own
// two 16-position halo blocks in registers, already in the MFMA B-fragment layout of the 1x1's
// f32 instruction sequence (lane group g holds channels 16 c + 4 g .. 16 c + 4 g + 3 of K chunk
// c), and every wave computes all channels of a slice for its 32 positions. The weights of each
// slice arrive by direct global -> LDS loads issued one phase ahead. The arithmetic is the f32
// unfused kernels' instruction for instruction: LayerNorm as k_layer_norm (f64 sums in channel
// order per position), the 1x1 convs as conv1x1_ring (bias, then v_mfma_f32_16x16x4_f32 over K
// chunks of 16 channels in ascending order), the depthwise 3x3 and gate as k_depthwise3x3, so the
// fused and unfused f32 paths agree bit for bit.

namespace {

typedef float f32x2 __attribute__((ext_vector_type(2)));

__device__ u32x4 g_zero_ffn32[8];  // 128 zero bytes: the source of absent biases

// s_waitcnt vmcnt(N) (expcnt and lgkmcnt not waited for); gfx9 splits vmcnt over [3:0] and [15:14].
template <int N>
__device__ __forceinline__ void ffn_wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// LayerNorm of this wave's halo positions into B fragments: u[i][c] holds channels
// 16 c + 4 grp .. + 3 of halo position (2 wave + i) * 16 + col. Statistics as k_layer_norm: one
// thread per halo position sums its channels in order in f64 (positions outside the picture
// read zeros; their values are never used, the 1x1's output is zeroed there). Ends after the
// statistics barrier; the caller's direct loads issued before it are waited for by the loads here.
template <int DIM>
__device__ __forceinline__ void ln_frags_f32(const float* xb, const View& xv, int y0, int x0, int h, int w,
                                             const float* ln_w, const float* ln_b, float* s_stat, int tid,
                                             int wave, int col, int grp, f32x4 (&u)[2][DIM / 16]) {
    constexpr int NCH = DIM / 16;
    if (tid < FNP) {
        const int iy = y0 - 1 + tid / FH, ix = x0 - 1 + tid % FH;
        double mean = 0.0, var = 0.0;
        if (iy >= 0 && iy < h && ix >= 0 && ix < w) {
            const float* r = xb + (long long)iy * xv.row + (long long)ix * xv.cs;
#pragma unroll 8
            for (int q = 0; q < DIM / 4; ++q) {
                const f32x4 v = *(const f32x4*)(r + 4 * q);
#pragma unroll
                for (int k = 0; k < 4; ++k) mean += (double)v[k];
            }
            mean /= (double)DIM;
#pragma unroll 8
            for (int q = 0; q < DIM / 4; ++q) {
                const f32x4 v = *(const f32x4*)(r + 4 * q);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const double e = (double)v[k] - mean;
                    var = var + e * e;
                }
            }
        } else {
            mean /= (double)DIM;
            var = 0.0;
        }
        s_stat[tid] = (float)mean;
        s_stat[FNP + tid] = sqrtf((float)(var / (double)DIM) + 1e-5f);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int pos = (2 * wave + i) * 16 + col;
        const int iy = y0 - 1 + pos / FH, ix = x0 - 1 + pos % FH;
        const bool inside = iy >= 0 && iy < h && ix >= 0 && ix < w;
        const float* r = xb + (long long)iy * xv.row + (long long)ix * xv.cs + 4 * grp;
#pragma unroll
        for (int c = 0; c < NCH; ++c) u[i][c] = inside ? *(const f32x4*)(r + 16 * c) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int pos = (2 * wave + i) * 16 + col;
        const float m = s_stat[pos], d = s_stat[FNP + pos];
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const f32x4 lw = *(const f32x4*)(ln_w + 16 * c + 4 * grp);
            const f32x4 lb = *(const f32x4*)(ln_b + 16 * c + 4 * grp);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                float e = u[i][c][k] - m;
                e = e / d;
                e = e * lw[k];
                u[i][c][k] = e + lb[k];
            }
        }
    }
}

// acc[cb][i] = bias + W (64 rows: four 16-row blocks in LDS as [chunk][block][16][4 units], unit q
// of row r at q ^ gswz(r)) x u for this wave's two position blocks, the 1x1's f32 instruction
// sequence.
template <int NCH>
__device__ __forceinline__ void slice_gemm_f32(const u32x4* s_w, const float* bias64, const f32x4 (&u)[2][NCH],
                                               int col, int grp, f32x4 (&acc)[4][2]) {
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
        const f32x4 bi = *(const f32x4*)(bias64 + cb * 16 + 4 * grp);
        acc[cb][0] = bi;
        acc[cb][1] = bi;
    }
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        // One chunk's 16 weight registers at a time (32 MFMAs cover the LDS latency); without the
        // fence the compiler hoists every chunk's reads and spills.
        __builtin_amdgcn_sched_barrier(0);
        f32x4 a[4];
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) a[cb] = __builtin_bit_cast(f32x4, s_w[(c * 4 + cb) * 64 + col * 4 + (grp ^ gswz(col))]);
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int cb = 0; cb < 4; ++cb)
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    acc[cb][i] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[cb][k], u[i][c][k], acc[cb][i], 0, 0, 0);
    }
}

}  // namespace

// Feed-forward, f32: as k_ffn, slices of 32 gate pairs (64 p channels). LDS: W_in slice
// [chunk][4 blocks][16][4] (32 KB at dim 128), p [256 positions][64] (a and b halves swapped on
// odd positions, 16-byte units XORed with pos & 7 so that the project_in stores of 8
// neighbouring positions -- one 8-lane ds_write_b128 pass over 128 bytes of banks -- are
// conflict-free), g [208 positions][32] (units XORed with 2 ((pos >> 1) & 3): conflict-free
// fragment reads), W_out slice [2 chunks][dim / 16 blocks][16][4], and per slice b_in, the
// depthwise taps and biases. The weight rows take gswz.
template <int DIM>
__global__ void __launch_bounds__(FTHREADS) k_ffn_f32(const FfnArgs p) {
    constexpr int HID = 4 * DIM, C2 = 2 * HID, NS = HID / 32, NCH = DIM / 16;
    constexpr int CB2 = DIM / 16, WPC = 8 / CB2, NPB = (FPB + WPC - 1) / WPC;
    constexpr int WIN_U = NCH * 4 * 64, P_U = FNP * 16, G_U = FPB * 16 * 8, WO_U = 2 * CB2 * 64;
    constexpr int X_U = 11 * 16;  // b_in [64], depthwise taps [9][64], depthwise bias [64] (f32)
    constexpr int WIN_W = NCH * 4 / 8, WO_W = 2 * CB2 / 8;  // direct loads per wave and slice
    static_assert(WIN_W * 8 == NCH * 4 && WO_W * 8 == 2 * CB2, "load shapes");
    static_assert(FOP <= FPB * 16 && 2 * 8 * 16 == FNP, "tile shapes");
    // One LDS object per buffer: the compiler then sees that the direct loads into one buffer
    // cannot alias the reads of another and waits for them only where this code does.
    __shared__ u32x4 s_win[WIN_U];
    __shared__ float s_p[P_U * 4];
    __shared__ float s_g[G_U * 4];
    __shared__ u32x4 s_wo[WO_U];
    __shared__ u32x4 s_x[2 * X_U];
    __shared__ float s_stat[2 * FNP];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int bid = (int)blockIdx.x;
    const int tx = bid % p.gx, ty = (bid / p.gx) % p.gy, b = bid / (p.gx * p.gy);
    const int y0 = ty * FT, x0 = tx * FT;
    const float* xb = (const float*)p.x.p + (long long)b * p.x.bstride + p.x.c_off;
    const u32x4* w_in = (const u32x4*)p.w_in;
    const u32x4* w_out = (const u32x4*)p.w_out;

    // Slice s weights. W_in block (c, cb): 16 rows of p channels 32 s + 16 cb (cb < 2) or
    // hid + 32 s + 16 (cb - 2), K chunk c: one contiguous KB of the packed weight.
    auto issue_win = [&](int s) {
#pragma unroll
        for (int j = 0; j < WIN_W; ++j) {
            const int blk = wave + 8 * j, c = blk >> 2, cb = blk & 3;
            const int gb = cb < 2 ? 2 * s + cb : HID / 16 + 2 * s + (cb - 2);
            lds_dma16(w_in + ((long long)c * p.nblk_in + gb) * 64 + (lane ^ gswz(lane >> 2)), s_win + blk * 64);
        }
    };
    auto issue_wout = [&](int s) {  // K chunks 2 s, 2 s + 1: 2 CB2 contiguous KB
#pragma unroll
        for (int j = 0; j < WO_W; ++j) {
            const int blk = wave + 8 * j;
            lds_dma16(w_out + ((long long)2 * s * p.nblk_out + blk) * 64 + (lane ^ gswz(lane >> 2)), s_wo + blk * 64);
        }
    };
    // Unit u of X (176): run u / 8 of 32 floats; runs 0-1 b_in, 2-19 tap (run - 2) / 2, 20-21 the
    // depthwise bias; even runs the first-half channels 32 s .., odd runs hid + 32 s ...
    auto issue_x = [&](int s, int buf) {
        if (wave < 3) {
            const int u = wave * 64 + lane;
            if (u < X_U) {
                const int run = u >> 3, half = run & 1, q = u & 7;
                const int ch = (half ? HID : 0) + 32 * s + 4 * q;
                const void* src;
                if (run < 2) src = p.b_in ? (const void*)(p.b_in + ch) : (const void*)(g_zero_ffn32 + q);
                else if (run < 20) src = p.dw_w + ((run - 2) >> 1) * C2 + ch;
                else src = p.dw_b ? (const void*)(p.dw_b + ch) : (const void*)(g_zero_ffn32 + q);
                lds_dma16(src, s_x + buf * X_U + wave * 64);
            }
        }
    };

    issue_win(0);
    issue_x(0, 0);
    f32x4 u[2][NCH];
    ln_frags_f32<DIM>(xb, p.x, y0, x0, p.h, p.w, p.ln_w, p.ln_b, s_stat, tid, wave, col, grp, u);

    const int cb2 = wave % CB2, pw2 = wave / CB2;
    f32x4 acc2[NPB];
    {
        f32x4 bo = {0.0f, 0.0f, 0.0f, 0.0f};
        if (p.b_out) bo = *(const f32x4*)(p.b_out + cb2 * 16 + 4 * grp);
#pragma unroll
        for (int i = 0; i < NPB; ++i) acc2[i] = bo;
    }
    // Depthwise role (tid < 448, waves 0-6): gate pair pg of the slice, column dc, all rows.
    const int pg = tid & 31, dc = (tid >> 5) % FT;
    const bool dw_thread = tid < 32 * FT;

    for (int s = 0; s < NS; ++s) {
        ffn_wait_vmcnt<0>();
        __syncthreads();  // W_in(s), X(s) landed; p, g and the W_out buffer free
        issue_wout(s);
        if (s + 1 < NS) issue_x(s + 1, (s + 1) & 1);
        const float* sx = reinterpret_cast<const float*>(s_x + (s & 1) * X_U);

        // a. p slice = b_in + W_in x u for this wave's positions; zero outside the picture.
        {
            f32x4 acc1[4][2];
            slice_gemm_f32<NCH>(s_win, sx, u, col, grp, acc1);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int pos = (2 * wave + i) * 16 + col;
                const int iy = y0 - 1 + pos / FH, ix = x0 - 1 + pos % FH;
                const bool inside = iy >= 0 && iy < p.h && ix >= 0 && ix < p.w;
#pragma unroll
                for (int cb = 0; cb < 4; ++cb) {
                    const int half = (cb >> 1) ^ (col & 1);  // pos & 1 == col & 1
                    const f32x4 v = inside ? acc1[cb][i] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                    const int unit = (half * 8 + (cb & 1) * 4 + grp) ^ (col & 7);  // pos & 7 == col & 7
                    *(f32x4*)(s_p + pos * 64 + unit * 4) = v;
                }
            }
        }
        __syncthreads();  // p ready; W_in(s) consumed

        // b. depthwise 3x3 + ELU gate (k_depthwise3x3's order: bias, then taps (ky, kx) ascending).
        if (dw_thread) {
            const float* dww = sx + 64;
            float wa[9], wb[9];
            const float ba = dww[576 + pg], bb = dww[576 + 32 + pg];
#pragma unroll
            for (int tp = 0; tp < 9; ++tp) {
                wa[tp] = dww[tp * 64 + pg];
                wb[tp] = dww[tp * 64 + 32 + pg];
            }
            // p row of halo position (hr, dc + kx): hr * FH + dc + kx, its two 32-channel halves
            // swapped on odd positions and its 16-byte units XORed with pos & 7. FH = 16, so both
            // depend on dc + kx only and each read is a fixed per-kx offset plus hr rows
            // (immediate offsets once the rows unroll).
            int offa[3], offb[3];
#pragma unroll
            for (int kx = 0; kx < 3; ++kx) {
                const int c = dc + kx, odd = c & 1, sw = c & 7;
                offa[kx] = c * 64 + ((odd * 8 + (pg >> 2)) ^ sw) * 4 + (pg & 3);
                offb[kx] = c * 64 + (((odd ^ 1) * 8 + (pg >> 2)) ^ sw) * 4 + (pg & 3);
            }
            static_assert(FH == 16, "row swizzle");
            auto ld = [&](int hr, int kx, float& oa, float& ob) {
                oa = s_p[hr * (FH * 64) + offa[kx]];
                ob = s_p[hr * (FH * 64) + offb[kx]];
            };
            float xa[3][3], xq[3][3];
#pragma unroll
            for (int kx = 0; kx < 3; ++kx) {
                ld(0, kx, xa[0][kx], xq[0][kx]);
                ld(1, kx, xa[1][kx], xq[1][kx]);
            }
#pragma unroll
            for (int oy = 0; oy < FT; ++oy) {
#pragma unroll
                for (int kx = 0; kx < 3; ++kx) ld(oy + 2, kx, xa[2][kx], xq[2][kx]);
                float a = ba, bq = bb;
#pragma unroll
                for (int ky = 0; ky < 3; ++ky)
#pragma unroll
                    for (int kx = 0; kx < 3; ++kx) {
                        a = fmaf(wa[ky * 3 + kx], xa[ky][kx], a);
                        bq = fmaf(wb[ky * 3 + kx], xq[ky][kx], bq);
                    }
                const float e = cephes_exp(a) - 1.0f;
                const float elu = a > 0.0f ? a : e;
                const int o = oy * FT + dc;
                s_g[o * 32 + (((pg >> 2) ^ (((o >> 1) & 3) << 1)) << 2) + (pg & 3)] = elu * bq;
#pragma unroll
                for (int kx = 0; kx < 3; ++kx) {
                    xa[0][kx] = xa[1][kx];
                    xa[1][kx] = xa[2][kx];
                    xq[0][kx] = xq[1][kx];
                    xq[1][kx] = xq[2][kx];
                }
            }
        }
        // W_in(s + 1) flies during phase c. W_out(s), issued before it, has landed once at most
        // WIN_W loads are pending.
        if (s + 1 < NS) issue_win(s + 1);
        if (s + 1 < NS) ffn_wait_vmcnt<WIN_W>();
        else ffn_wait_vmcnt<0>();
        __syncthreads();  // g ready; W_out(s) landed

        // c. y += W_out(s) x g: K chunks 2 s, 2 s + 1 (channel 16 cc + 4 grp + k of the slice).
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            const f32x4 a = __builtin_bit_cast(f32x4, s_wo[(cc * CB2 + cb2) * 64 + col * 4 + (grp ^ gswz(col))]);
            // The g swizzle depends on bits 1-2 of the position, i.e. of col: one base address.
            const float* gq = s_g + (pw2 * 16 + col) * 32 + (((cc * 4 + grp) ^ (((col >> 1) & 3) << 1)) << 2);
            // Position blocks in groups of GB (fewer live fragment registers).
            constexpr int GB = 7;
#pragma unroll
            for (int i0 = 0; i0 < NPB; i0 += GB) {
                __builtin_amdgcn_sched_barrier(0);
                f32x4 bv[GB];
#pragma unroll
                for (int j = 0; j < GB; ++j)
                    if (i0 + j < NPB && pw2 + WPC * (i0 + j) < FPB) bv[j] = *(const f32x4*)(gq + WPC * (i0 + j) * 512);
#pragma unroll
                for (int k = 0; k < 4; ++k)
#pragma unroll
                    for (int j = 0; j < GB; ++j)
                        if (i0 + j < NPB && pw2 + WPC * (i0 + j) < FPB)
                            acc2[i0 + j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[k], bv[j][k], acc2[i0 + j], 0, 0, 0);
            }
        }
    }

    // ---- 3. y = acc + x, stored from the fragments (16 bytes per lane, 64-byte channel runs).
    float* yb = (float*)p.y.p + (long long)b * p.y.bstride + p.y.c_off;
#pragma unroll
    for (int i = 0; i < NPB; ++i) {
        const int pb = pw2 + WPC * i, pos = pb * 16 + col;
        if (pb >= FPB || pos >= FOP) continue;
        const int oy = y0 + pos / FT, ox = x0 + pos % FT;
        if (oy >= p.h || ox >= p.w) continue;
        const int ch = cb2 * 16 + 4 * grp;
        const f32x4 r = *(const f32x4*)(xb + (long long)oy * p.x.row + (long long)ox * p.x.cs + ch);
        f32x4 v = acc2[i];
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = v[k] + r[k];
        *(f32x4*)(yb + (long long)oy * p.y.row + (long long)ox * p.y.cs + ch) = v;
    }
}

// prep_data, f32: as k_qkv, slices of 64 of the 3 dim conv1 channels; the 1x1 as in k_ffn_f32,
// p [256 positions][64] in LDS, the depthwise stored straight to qkv. The biases and depthwise
// taps of every slice (17 KB at dim 128) are loaded once, with the first slice's weights.
template <int DIM>
__global__ void __launch_bounds__(FTHREADS) k_qkv_f32(const QkvArgs p) {
    // p rows swizzled (16-byte units XORed with pos & 15) at dim 128 only: at dim 64 the
    // compiler then renamed MFMA accumulator chains closer than the ISA guard allows.
    constexpr int PSWZ = DIM == 128 ? 15 : 0;
    constexpr int C3 = 3 * DIM, NS = C3 / 64, NCH = DIM / 16;
    constexpr int W1_U = NCH * 4 * 64, P_U = FNP * 16, X_U = 11 * 16;
    constexpr int W1_W = NCH * 4 / 8;
    static_assert(W1_W * 8 == NCH * 4 && C3 % 64 == 0, "load shapes");
    __shared__ u32x4 s_w1[W1_U];
    __shared__ float s_p[P_U * 4];
    __shared__ u32x4 s_x[NS * X_U];
    __shared__ float s_stat[2 * FNP];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int bid = (int)blockIdx.x;
    const int tx = bid % p.gx, ty = (bid / p.gx) % p.gy, b = bid / (p.gx * p.gy);
    const int y0 = ty * FT, x0 = tx * FT;
    const float* xb = (const float*)p.x.p + (long long)b * p.x.bstride + p.x.c_off;
    const u32x4* w1 = (const u32x4*)p.w1;

    // Slice s: conv1 output channels 64 s .. 64 s + 63 (blocks 4 s .. 4 s + 3).
    auto issue_w1 = [&](int s) {
#pragma unroll
        for (int j = 0; j < W1_W; ++j) {
            const int blk = wave + 8 * j, c = blk >> 2, cb = blk & 3;
            lds_dma16(w1 + ((long long)c * p.nblk1 + 4 * s + cb) * 64 + (lane ^ gswz(lane >> 2)), s_w1 + blk * 64);
        }
    };
    // Unit u of slice s's X (176): run u / 16 of 64 floats; run 0 b1, 1-9 tap run - 1, 10 the
    // depthwise bias. Wave w loads 64-unit pieces w, w + 8, ... of all NS * 176 units.
    for (int j = wave; j * 64 < NS * X_U; j += 8) {
        const int v = j * 64 + lane;
        if (v < NS * X_U) {
            const int s = v / X_U, u = v - s * X_U;
            const int run = u >> 4, q = u & 15;
            const int ch = 64 * s + 4 * q;
            const void* src;
            if (run == 0) src = p.b1 ? (const void*)(p.b1 + ch) : (const void*)(g_zero_ffn32 + (q & 7));
            else if (run < 10) src = p.dw_w + (run - 1) * C3 + ch;
            else src = p.dw_b ? (const void*)(p.dw_b + ch) : (const void*)(g_zero_ffn32 + (q & 7));
            lds_dma16(src, s_x + j * 64);
        }
    }
    issue_w1(0);
    f32x4 u[2][NCH];
    ln_frags_f32<DIM>(xb, p.x, y0, x0, p.h, p.w, p.ln_w, p.ln_b, s_stat, tid, wave, col, grp, u);

    // Depthwise role (tid < 448, waves 0-6): channel pair pg of the slice, column dc, all rows.
    const int pg = tid & 31, dc = (tid >> 5) % FT;
    const bool dw_thread = tid < 32 * FT;
    float* yb = (float*)p.y.p + (long long)b * p.y.bstride + p.y.c_off;

    for (int s = 0; s < NS; ++s) {
        ffn_wait_vmcnt<0>();
        __syncthreads();  // W1(s) landed; p free
        const float* sx = reinterpret_cast<const float*>(s_x + s * X_U);
        {
            f32x4 acc1[4][2];
            slice_gemm_f32<NCH>(s_w1, sx, u, col, grp, acc1);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int pos = (2 * wave + i) * 16 + col;
                const int iy = y0 - 1 + pos / FH, ix = x0 - 1 + pos % FH;
                const bool inside = iy >= 0 && iy < p.h && ix >= 0 && ix < p.w;
#pragma unroll
                for (int cb = 0; cb < 4; ++cb)  // the row's 16 units XORed with pos & 15 (bank spread)
                    *(f32x4*)(s_p + pos * 64 + (((cb * 4 + grp) ^ (pos & PSWZ)) << 2)) =
                        inside ? acc1[cb][i] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            }
        }
        __syncthreads();  // p ready; W1(s) consumed
        if (s + 1 < NS) issue_w1(s + 1);
        if (dw_thread) {
            const float* dww = sx + 64;
            float wv[9][2], bv[2];
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                bv[k] = dww[576 + 2 * pg + k];
#pragma unroll
                for (int tp = 0; tp < 9; ++tp) wv[tp][k] = dww[tp * 64 + 2 * pg + k];
            }
            float xw[3][3][2];
            // The swizzle pos & PSWZ of halo position (hr, dc + kx) is (dc + kx) & PSWZ (PSWZ < FH,
            // FH a power of two), so each read is a per-kx offset plus hr rows.
            static_assert(PSWZ < FH && (FH & (FH - 1)) == 0, "row swizzle");
            int off[3];
#pragma unroll
            for (int kx = 0; kx < 3; ++kx)
                off[kx] = (dc + kx) * 64 + ((((pg >> 1) ^ ((dc + kx) & PSWZ)) << 2) + 2 * (pg & 1));
            auto ld = [&](int hr, int kx, float (&o)[2]) {
                const f32x2 v = *(const f32x2*)(s_p + hr * (FH * 64) + off[kx]);
                o[0] = v[0];
                o[1] = v[1];
            };
#pragma unroll
            for (int kx = 0; kx < 3; ++kx) {
                ld(0, kx, xw[0][kx]);
                ld(1, kx, xw[1][kx]);
            }
            const int ox = x0 + dc;
#pragma unroll
            for (int r = 0; r < FT; ++r) {
#pragma unroll
                for (int kx = 0; kx < 3; ++kx) ld(r + 2, kx, xw[2][kx]);
                float o[2];
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    float a = bv[k];
#pragma unroll
                    for (int ky = 0; ky < 3; ++ky)
#pragma unroll
                        for (int kx = 0; kx < 3; ++kx) a = fmaf(wv[ky * 3 + kx][k], xw[ky][kx][k], a);
                    o[k] = a;
                }
                const int oy = y0 + r;
                if (oy < p.h && ox < p.w)
                    *(f32x2*)(yb + (long long)oy * p.y.row + (long long)ox * p.y.cs + 64 * s + 2 * pg) = f32x2{o[0], o[1]};
#pragma unroll
                for (int kx = 0; kx < 3; ++kx)
#pragma unroll
                    for (int k = 0; k < 2; ++k) {
                        xw[0][kx][k] = xw[1][kx][k];
                        xw[1][kx][k] = xw[2][kx][k];
                    }
            }
        }
    }
}

bool qkv_fused_supported(int dtype, int dim) {
    return (dtype == DT_F32 || dtype == DT_F16 || dtype == DT_BF16) && (dim == 64 || dim == 128);
}

hipError_t launch_qkv_fused(const QkvArgs& a, int dtype, int dim, hipStream_t s) {
    if (!qkv_fused_supported(dtype, dim)) return hipErrorInvalidValue;
    // 16-byte loads of x (4 f32 or 8 16-bit channels), 2-channel stores of y.
    const int xv = dtype == DT_F32 ? 4 : 8;
    if (a.x.cs % xv || a.x.c_off % xv || a.x.row % xv || a.x.bstride % xv || a.y.cs % 2 || a.y.c_off % 2 ||
        a.y.row % 2 || a.y.bstride % 2)
        return hipErrorInvalidValue;
    if (a.N <= 0 || a.h <= 0 || a.w <= 0) return hipSuccess;
    QkvArgs p = a;
    p.gx = (a.w + FT - 1) / FT;
    p.gy = (a.h + FT - 1) / FT;
    const long long blocks = (long long)p.gx * p.gy * a.N;
    if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
    const dim3 grid((unsigned)blocks), block(FTHREADS);
    if (dtype == DT_F32) {
        if (dim == 128) k_qkv_f32<128><<<grid, block, 0, s>>>(p);
        else k_qkv_f32<64><<<grid, block, 0, s>>>(p);
    } else if (dtype == DT_BF16) {
        if (dim == 128) k_qkv<__bf16, 128><<<grid, block, 0, s>>>(p);
        else k_qkv<__bf16, 64><<<grid, block, 0, s>>>(p);
    } else {
        if (dim == 128) k_qkv<_Float16, 128><<<grid, block, 0, s>>>(p);
        else k_qkv<_Float16, 64><<<grid, block, 0, s>>>(p);
    }
    return hipGetLastError();
}

bool ffn_fused_supported(int dtype, int dim) {
    return (dtype == DT_F32 || dtype == DT_F16 || dtype == DT_BF16) && (dim == 64 || dim == 128);
}

hipError_t launch_ffn_fused(const FfnArgs& a, int dtype, int dim, hipStream_t s) {
    if (!ffn_fused_supported(dtype, dim)) return hipErrorInvalidValue;
    // 16-byte vector accesses of x and y (4 f32 or 8 16-bit channels).
    const int v = dtype == DT_F32 ? 4 : 8;
    if (a.x.cs % v || a.x.c_off % v || a.x.row % v || a.x.bstride % v || a.y.cs % v || a.y.c_off % v ||
        a.y.row % v || a.y.bstride % v)
        return hipErrorInvalidValue;
    if (a.N <= 0 || a.h <= 0 || a.w <= 0) return hipSuccess;
    FfnArgs p = a;
    p.gx = (a.w + FT - 1) / FT;
    p.gy = (a.h + FT - 1) / FT;
    const long long blocks = (long long)p.gx * p.gy * a.N;
    if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
    const dim3 grid((unsigned)blocks), block(FTHREADS);
    if (dtype == DT_F32) {
        if (dim == 128) k_ffn_f32<128><<<grid, block, 0, s>>>(p);
        else k_ffn_f32<64><<<grid, block, 0, s>>>(p);
    } else if (dtype == DT_BF16) {
        if (dim == 128) k_ffn<__bf16, 128><<<grid, block, 0, s>>>(p);
        else k_ffn<__bf16, 64><<<grid, block, 0, s>>>(p);
    } else {
        if (dim == 128) k_ffn<_Float16, 128><<<grid, block, 0, s>>>(p);
        else k_ffn<_Float16, 64><<<grid, block, 0, s>>>(p);
    }
    return hipGetLastError();
}

}  // namespace zjai
