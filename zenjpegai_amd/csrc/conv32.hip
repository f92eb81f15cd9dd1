// Dense stride-1 3x3 convolutions in f16 / bf16 with 64 or 128 input channels on gfx950's
// v_mfma_f32_32x32x16.
//
// One workgroup of 4 waves computes all MT output channels of a channel tile (MT = 128 or 64)
// for 256 output positions (TR rows x TW columns, TW = 32 or 16). The input halo
// [TR + 2][TW + 2][all input channels] is loaded into LDS once, with direct global -> LDS loads
// (global_load_lds_dwordx4: lane i's 16 bytes land at the wave's LDS base + 16 i, no VGPR
// staging) that read each pixel's channels as one contiguous run (padding units load from a
// zeroed device buffer); the 16-byte slots of a pixel are XOR-swizzled by the pixel index so
// the fragment reads are free of bank conflicts. The weights stream through LDS 16 input
// channels at a time ([9][2][MT][8]), double-buffered: one barrier per chunk, the next chunk's
// loads in flight during this chunk's MFMAs. Wave w owns positions [64 w, 64 w + 64) as two
// 32-position B fragments and all MT / 32 A fragments.
//
// MFMA lane map (32x32x16): lane (j, h) = (lane % 32, lane / 32) supplies row / column j and
// channels 8h..8h+7 of the 16-channel step; accumulator register r holds output channel
// 8 (r / 4) + 4 h + r % 4 of the A fragment, at position j of the B fragment.
// Per output the sum runs bias first, then chunk by chunk, tap by tap (ky, kx ascending), 16
// channels per MFMA; the epilogue is the shared one (epilogue.h) through an LDS transpose, so
// every position's channels leave as one contiguous run.

#include "conv.h"
#include "epilogue.h"
#include "mfma.h"

namespace zjai {

__device__ u32x4 g_zero_units32[4];  // 64 zero bytes: the source of padding units

template <typename T, int MT, int TW, int S>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
conv3x3_m32(const ConvParams p) {
    constexpr int NT = 256;
    constexpr int TR = 256 / TW;
    constexpr int HR = TR + 2, HC = TW + 2;
    constexpr int MA = MT / 32;
    constexpr int NPIX = HR * HC;
    constexpr int HALO_U = NPIX * S;  // [pixel][S 16-byte slots], slot s holds unit s ^ (pixel % S)
    constexpr int W_U = 9 * MT * 2;   // one 16-channel chunk: [tap][half][MT] 16-byte units
    constexpr int MAIN_U = HALO_U + 2 * W_U;
    constexpr int OUT_LD = MT + 4;    // f32 per transposed position (+4: fewer bank conflicts)
    constexpr int NPASS = (256 * OUT_LD > MAIN_U * 4) ? 2 : 1;
    constexpr int PPASS = 256 / NPASS;
    constexpr int OUT_U = (PPASS * OUT_LD + 3) / 4;
    constexpr int LDS_U = MAIN_U > OUT_U ? MAIN_U : OUT_U;
    constexpr int HN = (HALO_U + NT - 1) / NT, WN = (W_U + NT - 1) / NT;
    static_assert(MT % 32 == 0 && (TW == 16 || TW == 32) && (S == 8 || S == 16), "tile");
    __shared__ u32x4 s_lds[LDS_U];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j = lane & 31, h = lane >> 5;

    // XCD-aware order (conv.hip's scheme): logical order (batch, tile row, tile col, channel
    // tile), the channel tiles of one spatial tile consecutive on one XCD (shared halo in L2).
    const int nmt = p.ntiles;
    const int total = p.gx * p.gy * p.N * nmt;
    const int bid = (int)blockIdx.x, xj = bid & 7, xk = bid >> 3;
    const int q8 = total >> 3, r8 = total & 7;
    const int lid = xj < r8 ? xj * (q8 + 1) + xk : r8 * (q8 + 1) + (xj - r8) * q8 + xk;
    int rest = lid / nmt;
    const int mt = lid - rest * nmt;
    const int tx = rest % p.gx;
    rest /= p.gx;
    const int ty = rest % p.gy, bi = rest / p.gy;
    const int ox0 = tx * TW, oy0 = ty * TR;
    const int oc0 = mt * MT;

    f32x16 acc[MA][2];
#pragma unroll
    for (int a = 0; a < MA; ++a) {
        f32x16 b;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int oc = oc0 + 32 * a + 8 * (r >> 2) + 4 * h + (r & 3);
            b[r] = (p.bias && oc < p.cout_g) ? p.bias[oc] : 0.0f;
        }
        acc[a][0] = b;
        acc[a][1] = b;
    }

    const T* xg = (const T*)p.x.p + (long long)bi * p.x.bstride + p.x.c_off;
    const u32x4* wg = (const u32x4*)p.w + (long long)mt * W_U;
    const long long wchunk = (long long)nmt * W_U;
    u32x4* s_halo = s_lds;
    u32x4* s_wt = s_lds + HALO_U;

    // The whole halo (all S * 8 input channels) once: LDS unit U = pixel * S + slot takes the
    // pixel's channel unit slot ^ (pixel % S), so each pixel's S * 16 bytes are read as one
    // contiguous run (S lanes) while the fragment reads below hit S different bank groups.
#pragma unroll 4
    for (int i = 0; i < HN; ++i) {
        const int ub = wave * 64 + i * NT;
        if (ub >= HALO_U) break;
        const int U = ub + lane;
        if (U < HALO_U) {
            const int pix = U / S, slot = U - pix * S, cu = slot ^ (pix & (S - 1));
            const int hy = pix / HC, hx = pix - hy * HC;
            const int iy = oy0 - 1 + hy, ix = ox0 - 1 + hx;
            const void* src = (iy >= 0 && iy < p.H && ix >= 0 && ix < p.W)
                                  ? (const void*)(xg + (long long)iy * p.x.row + (long long)ix * p.x.cs + cu * 8)
                                  : (const void*)g_zero_units32;
            lds_dma16(src, s_halo + ub);
        }
    }
    auto issue_w = [&](int chunk, int buf) __attribute__((always_inline)) {
        const u32x4* wsrc = wg + chunk * wchunk;
        u32x4* dst = s_wt + buf * W_U;
#pragma unroll
        for (int i = 0; i < WN; ++i) {
            const int ub = wave * 64 + i * NT;
            if (ub >= W_U) break;
            if (ub + lane < W_U)
                lds_dma16(wsrc + ub + lane, dst + ub);
        }
    };

    // Halo pixel of this lane's position in B fragment b (before the tap offset).
    int hpix[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        const int pos = wave * 64 + 32 * b + j;
        hpix[b] = (pos / TW) * HC + pos % TW;
    }

    const int nchunks = p.nchunks;
    issue_w(0, 0);
    for (int c = 0; c < nchunks; ++c) {
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's loads of chunk c are in LDS
        __syncthreads();                     // ... and every other wave's
        if (c + 1 < nchunks) issue_w(c + 1, (c + 1) & 1);
        const u32x4* s_w = s_wt + (c & 1) * W_U + h * MT + j;
        const int cu = 2 * c + h;  // this lane's channel unit of the chunk
        u32x4 av[2][MA], bv[2][2];
        auto fetch = [&](int t, int set) __attribute__((always_inline)) {
            const int ky = t / 3, kx = t - 3 * (t / 3);
#pragma unroll
            for (int a = 0; a < MA; ++a) av[set][a] = s_w[t * 2 * MT + 32 * a];
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const int pp = hpix[b] + ky * HC + kx;
                bv[set][b] = s_halo[pp * S + (cu ^ (pp & (S - 1)))];
            }
        };
        fetch(0, 0);
#pragma unroll
        for (int t = 0; t < 9; ++t) {
            // Scheduling fences: the next tap's LDS reads issue before this tap's MFMAs, so their
            // latency hides behind 2 * MA MFMAs instead of stalling each one.
            if (t + 1 < 9) fetch(t + 1, (t + 1) & 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int a = 0; a < MA; ++a)
#pragma unroll
                for (int b = 0; b < 2; ++b) Mma32<T>::run(acc[a][b], av[t & 1][a], bv[t & 1][b]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // Epilogue through LDS, NPASS passes of PPASS positions.
    float* so = reinterpret_cast<float*>(s_lds);
    constexpr int QP = MT / 4;
#pragma unroll
    for (int pass = 0; pass < NPASS; ++pass) {
        __syncthreads();
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int pos = wave * 64 + 32 * b + j;
            if (pos / PPASS != pass) continue;
            float* d = so + (pos - pass * PPASS) * OUT_LD + 4 * h;
#pragma unroll
            for (int a = 0; a < MA; ++a)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    f32x4 v;
#pragma unroll
                    for (int i = 0; i < 4; ++i) v[i] = acc[a][b][4 * q + i];
                    *reinterpret_cast<f32x4*>(d + 32 * a + 8 * q) = v;
                }
        }
        __syncthreads();
        if (epilogue_simple(p)) {
            // 8 channels per thread and step (MT is a multiple of 64 and divides cout), the steps
            // unrolled so that several LDS reads are in flight.
            constexpr int QP8 = MT / 8;
#pragma unroll 4
            for (int u = tid; u < PPASS * QP8; u += NT) {
                const int pl = u / QP8, c8 = u - pl * QP8;
                const int pos = pass * PPASS + pl;
                const int oy = oy0 + pos / TW, ox = ox0 + pos % TW;
                const f32x4 v0 = *reinterpret_cast<const f32x4*>(so + pl * OUT_LD + c8 * 8);
                const f32x4 v1 = *reinterpret_cast<const f32x4*>(so + pl * OUT_LD + c8 * 8 + 4);
                if (oy < p.OH && ox < p.OW) epilogue_store8<T>(p, bi, oy, ox, oc0 + c8 * 8, v0, v1);
            }
        } else {
            for (int u = tid; u < PPASS * QP; u += NT) {
                const int pl = u / QP, cq = u - pl * QP;
                const int pos = pass * PPASS + pl;
                const int oy = oy0 + pos / TW, ox = ox0 + pos % TW;
                const int oc = oc0 + cq * 4;
                if (oy >= p.OH || ox >= p.OW || oc >= p.cout_g) continue;
                const f32x4 v = *reinterpret_cast<const f32x4*>(so + pl * OUT_LD + cq * 4);
                epilogue_store<T>(p, bi, oy, ox, oc, min(4, p.cout_g - oc), v);
            }
        }
    }
}

template <typename T, int MT, int TW, int S>
static hipError_t go_m32(const ConvParams& p0, hipStream_t s) {
    constexpr int TR = 256 / TW;
    ConvParams p = p0;
    if (p.groups != 1 || p.cout_g % MT || p.cin_g != S * 8 || p.N < 1 || p.N > MAXB || p.ps != 1 ||
        p.out_mode != OUT_NHWC || p.relu6_in || p.w_bstride || (p.x.cs & 7) || (p.x.c_off & 7))
        return hipErrorInvalidValue;
    p.nchunks = p.cin_g / 16;
    p.ntiles = p.cout_g / MT;
    p.gx = (p.OW + TW - 1) / TW;
    p.gy = (p.OH + TR - 1) / TR;
    const long long total = (long long)p.gx * p.gy * p.N * p.ntiles;
    if (total <= 0 || total > (1ll << 30)) return hipErrorInvalidValue;
    hipLaunchKernelGGL((conv3x3_m32<T, MT, TW, S>), dim3((unsigned)total), dim3(256), 0, s, p);
    return hipGetLastError();
}

int conv3x3_m32_width(int OH, int OW) {
    // The tile width that wastes fewer computed positions at the map's right / bottom edges
    // (32 on ties).
    const long long a32 = (long long)((OW + 31) / 32) * 32 * ((OH + 7) / 8) * 8;
    const long long a16 = (long long)((OW + 15) / 16) * 16 * ((OH + 15) / 16) * 16;
    return a16 < a32 ? 16 : 32;
}

template <typename T, int S>
static hipError_t go_m32_s(int mt, int tw, const ConvParams& p, hipStream_t s) {
    if (mt == 128) return tw == 32 ? go_m32<T, 128, 32, S>(p, s) : go_m32<T, 128, 16, S>(p, s);
    if (mt == 64) return tw == 32 ? go_m32<T, 64, 32, S>(p, s) : go_m32<T, 64, 16, S>(p, s);
    return hipErrorInvalidValue;
}

template <typename T>
static hipError_t go_m32_t(int mt, int tw, const ConvParams& p, hipStream_t s) {
    if (p.cin_g == 128) return go_m32_s<T, 16>(mt, tw, p, s);
    if (p.cin_g == 64) return go_m32_s<T, 8>(mt, tw, p, s);
    return hipErrorInvalidValue;
}

hipError_t launch_conv3x3_m32(int dtype, int mt, int tw, const ConvParams& p, hipStream_t s) {
    if (tw != 16 && tw != 32) return hipErrorInvalidValue;
    switch (dtype) {
        case DT_F16: return go_m32_t<_Float16>(mt, tw, p, s);
        case DT_BF16: return go_m32_t<__bf16>(mt, tw, p, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace zjai
