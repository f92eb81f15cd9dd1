// Bandwidth-bound kernels: layout changes, elementwise ops, depthwise 3x3, layer norm and the
// reductions of channel attention. Element order and rounding follow the reference's
// `nn::fast::{layers, depthwise, math}` (each op a separate IEEE operation, FMA only where the
// reference's contract has one). Every kernel covers N batch items (tiles of one shape).

#include "ops.h"

#include <algorithm>

namespace zjai {

// Decomposes a flat index over [N][h][w][q] (q = channel quads, fastest).
struct Idx4 {
    int b, y, x, cq;
};
__device__ __forceinline__ Idx4 split(long long i, int h, int w, int q) {
    Idx4 r;
    r.cq = (int)(i % q);
    long long t = i / q;
    r.x = (int)(t % w);
    t /= w;
    r.y = (int)(t % h);
    r.b = (int)(t / h);
    return r;
}

// ------------------------------------------------------------------------------ layout moves
// One workgroup per run of PT_X positions of a row: every channel plane's PT_X floats are read
// as contiguous row segments into LDS (PT_C channels per pass, all of a pass's loads in flight
// before the first is used), then each thread writes one position's 4 channels, so consecutive
// threads write consecutive bytes of the NHWC row. Reading 4 channel planes per position
// instead (one 4-byte access per plane and lane) fetched each 128-byte line of the planes three
// times over.
constexpr int PT_X = 8, PT_C = 256, PT_L = PT_C * PT_X / 256;
// LDS holds a pass as [channel quad][PT_X + 1 positions][4 channels]: the position's quad is one
// 16-byte read, and the odd quad stride (PT_X + 1 units) spreads a pass's lanes over the banks.
template <typename T>
__global__ void __launch_bounds__(256) k_planar_to_nhwc(const float* src, int C, int LH, int LW, Windows win,
                                                        int N, int h, int w, View dst) {
    __shared__ f32x4 s_t[PT_C / 4 * (PT_X + 1)];
    // XCD-aware order: workgroup ids are dealt round-robin to the 8 XCDs (each with its own L2),
    // so consecutive logical runs -- which share 128-byte lines of every plane row -- are given
    // to one XCD (the grid is padded to a multiple of 8).
    const int ntx = (w + PT_X - 1) / PT_X, nrun = ntx * h * N;
    const int lid = ((int)blockIdx.x & 7) * ((int)gridDim.x >> 3) + ((int)blockIdx.x >> 3);
    if (lid >= nrun) return;
    const int bx = lid % ntx, by = (lid / ntx) % h, b = lid / (ntx * h);
    const int x0 = bx * PT_X, nx = min(PT_X, w - x0), tid = threadIdx.x;
    const float* row = src + (long long)(win.y0[b] + by) * LW + win.x0[b] + x0;
    const long long plane = (long long)LH * LW;
    for (int c0 = 0; c0 < C; c0 += PT_C) {
        const int cc = min(PT_C, C - c0);
        float v[PT_L];
#pragma unroll
        for (int k = 0; k < PT_L; ++k) {
            // Clamped (in-window) address, so the loads issue back to back without branches.
            const int i = tid + k * 256, c = min(i / PT_X, cc - 1), x = min(i % PT_X, nx - 1);
            v[k] = row[(c0 + c) * plane + x];
        }
#pragma unroll
        for (int k = 0; k < PT_L; ++k) {
            const int i = tid + k * 256, c = i / PT_X, x = i % PT_X;
            if (c < cc) s_t[(c / 4) * (PT_X + 1) + x][c % 4] = v[k];
        }
        __syncthreads();
        const int q = cc / 4;
        for (int i = tid; i < nx * q; i += 256) {
            const int x = i / q, cq = i % q;
            store4<T>(at_mut<T>(dst, b, by, x0 + x, c0 + cq * 4), s_t[cq * (PT_X + 1) + x]);
        }
        __syncthreads();
    }
}

template <typename T>
__global__ void k_nhwc_to_planar(View src, int N, int C, int h, int w, float* dst) {
    const int q = (C + 3) / 4;
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)N * h * w * q) return;
    // x fastest so the planar writes coalesce.
    const int x = (int)(i % w);
    long long r = i / w;
    const int y = (int)(r % h);
    r /= h;
    const int cq = (int)(r % q), b = (int)(r / q);
    for (int k = 0; k < 4; ++k) {
        const int c = cq * 4 + k;
        if (c < C) dst[(((long long)b * C + c) * h + y) * w + x] = to_f32(*at<T>(src, b, y, x, c));
    }
}

template <typename T>
__global__ void k_copy(View src, View dst, int N, int C, int h, int w) {
    const int q = C / 4;
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)N * h * w * q) return;
    const Idx4 d = split(i, h, w, q);
    store4<T>(at_mut<T>(dst, d.b, d.y, d.x, d.cq * 4), load4<T>(at<T>(src, d.b, d.y, d.x, d.cq * 4)));
}

template <typename T>
__global__ void k_pixel_shuffle(View src, View dst, int N, int C, int h, int w, int r) {
    const int q = C / 4, oh = h * r, ow = w * r;
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)N * oh * ow * q) return;
    const Idx4 d = split(i, oh, ow, q);
    const int y = d.y / r, dy = d.y - y * r, x = d.x / r, dx = d.x - x * r;
    f32x4 v;
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = to_f32(*at<T>(src, d.b, y, x, (d.cq * 4 + k) * r * r + dy * r + dx));
    store4<T>(at_mut<T>(dst, d.b, d.y, d.x, d.cq * 4), v);
}

// ---------------------------------------------------------------------------------- eltwise
template <typename T>
__global__ void k_eltwise(int op, View xv, View sv, int N, int C, int h, int w) {
    const int q = C / 4;
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)N * h * w * q) return;
    const Idx4 d = split(i, h, w, q);
    T* px = at_mut<T>(xv, d.b, d.y, d.x, d.cq * 4);
    f32x4 v = load4<T>(px);
    f32x4 s = {0, 0, 0, 0};
    if (op >= EL_ADD) s = load4<T>(at<T>(sv, d.b, d.y, d.x, d.cq * 4));
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
// Row-sliding: a thread owns one 16-byte channel vector (V = 4 f32 or 8 f16/bf16 channels) of
// DW_X consecutive output columns over DW_R consecutive output rows. It keeps a 3-row window of
// input vectors in registers and loads one new input row per output row, so every input vector
// is loaded once per thread instead of three times; the unrolled row loop lets the next row's
// loads issue before the current row's FMAs. Lanes run over channels (a wave's load reads a
// contiguous channel run). For the ELU-gated FFN variant the two halves of a wave compute the
// two channel halves (first half: lanes 0-31, second half: lanes 32-63, same vectors) and swap
// them across lanes before gating, so each lane holds one window.
constexpr int DW_R = 8;

template <typename T> struct Dw {
    static constexpr int V = 16 / (int)sizeof(T);  // channels per 16-byte vector
    static constexpr int X = sizeof(T) == 4 ? 4 : 2;  // output columns per thread
};

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <typename T>
__device__ __forceinline__ void dw_unpack(u32x4 v, float (&o)[Dw<T>::V]) {
    if constexpr (sizeof(T) == 4) {
        const f32x4 f = __builtin_bit_cast(f32x4, v);
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = f[i];
    } else {
        typedef T t8 __attribute__((ext_vector_type(8)));
        const t8 hv = __builtin_bit_cast(t8, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = (float)hv[i];
    }
}

// Input vector at (y, x), channels [c, c + nv) (nv < V only at a channel tail), zero outside.
template <typename T>
__device__ __forceinline__ u32x4 dw_load(const View& src, int b, int y, int x, int h, int w, int c,
                                         int nv, bool valid) {
    u32x4 v = {0u, 0u, 0u, 0u};
    if (!valid || y < 0 || y >= h || x < 0 || x >= w) return v;
    const T* px = at<T>(src, b, y, x, c);
    if (nv == Dw<T>::V) return *reinterpret_cast<const u32x4*>(px);
    T tmp[Dw<T>::V];
#pragma unroll
    for (int k = 0; k < Dw<T>::V; ++k) tmp[k] = k < nv ? px[k] : (T)0.0f;
    return __builtin_bit_cast(u32x4, tmp);
}

template <typename T>
__global__ void __launch_bounds__(256) k_depthwise3x3(View src, View dst, int N, int C, int h, int w,
                                                      const float* wt, const float* bias, int elu_half) {
    constexpr int V = Dw<T>::V, X = Dw<T>::X;
    const bool gated = elu_half > 0;
    const int cout = gated ? elu_half : C;
    const int nvec = (cout + V - 1) / V, vpw = gated ? 32 : 64, nvw = (nvec + vpw - 1) / vpw;
    const int lane = threadIdx.x & 63;
    // XCD-aware order: the hardware deals workgroups to the 8 XCDs round-robin, so workgroup p
    // takes logical block (p % 8) * (gridDim.x / 8) + p / 8 and each XCD works through one
    // contiguous run of column groups, whose overlapping input columns then meet in its L2.
    const long long nb8 = gridDim.x / 8;
    const long long blk = (blockIdx.x % 8) * nb8 + blockIdx.x / 8;
    const long long wave = (blk * blockDim.x + threadIdx.x) >> 6;
    const int gx = (w + X - 1) / X, gr = (h + DW_R - 1) / DW_R;
    if (wave >= (long long)N * gr * gx * nvw) return;  // whole waves only
    const int cw = (int)(wave % nvw);
    long long t = wave / nvw;
    const int xg = (int)(t % gx);
    t /= gx;
    const int rs = (int)(t % gr), b = (int)(t / gr);
    const int vidx = cw * vpw + (gated ? (lane & 31) : lane), half = gated ? lane >> 5 : 0;
    const bool valid = vidx < nvec;
    const int nv = valid ? min(V, cout - vidx * V) : 0;
    const int c0 = vidx * V + half * elu_half;  // channel of this lane's strip
    const int x0 = xg * X, y0 = rs * DW_R;

    float wv[9][V], bv[V];
#pragma unroll
    for (int k = 0; k < V; ++k) bv[k] = (bias && k < nv) ? bias[c0 + k] : 0.0f;
#pragma unroll
    for (int tp = 0; tp < 9; ++tp)
#pragma unroll
        for (int k = 0; k < V; ++k) wv[tp][k] = k < nv ? wt[tp * C + c0 + k] : 0.0f;

    u32x4 win[3][X + 2];
#pragma unroll
    for (int j = 0; j < X + 2; ++j) {
        win[0][j] = dw_load<T>(src, b, y0 - 1, x0 + j - 1, h, w, c0, nv, valid);
        win[1][j] = dw_load<T>(src, b, y0, x0 + j - 1, h, w, c0, nv, valid);
    }
#pragma unroll
    for (int r = 0; r < DW_R; ++r) {
        const int oy = y0 + r;
        if (oy >= h) break;  // uniform per wave
#pragma unroll
        for (int j = 0; j < X + 2; ++j) win[2][j] = dw_load<T>(src, b, oy + 1, x0 + j - 1, h, w, c0, nv, valid);
        float acc[X][V];
#pragma unroll
        for (int j = 0; j < X; ++j)
#pragma unroll
            for (int k = 0; k < V; ++k) acc[j][k] = bv[k];
#pragma unroll
        for (int ky = 0; ky < 3; ++ky) {
            float row[X + 2][V];
#pragma unroll
            for (int j = 0; j < X + 2; ++j) dw_unpack<T>(win[ky][j], row[j]);
            // Taps in (ky, kx) ascending order per output: acc = fma(w, x, acc).
#pragma unroll
            for (int j = 0; j < X; ++j)
#pragma unroll
                for (int kx = 0; kx < 3; ++kx)
#pragma unroll
                    for (int k = 0; k < V; ++k) acc[j][k] = fmaf(wv[ky * 3 + kx][k], row[j + kx][k], acc[j][k]);
        }
        if (gated) {
            // Lane l < 32 holds the first-half channels, lane l + 32 the matching second half.
#pragma unroll
            for (int j = 0; j < X; ++j)
#pragma unroll
                for (int k = 0; k < V; ++k) {
                    const float g = __shfl_xor(acc[j][k], 32);
                    const float v = acc[j][k];
                    float elu;
                    if constexpr (sizeof(T) == 4) {
                        const float e = cephes_exp(v) - 1.0f;
                        elu = v > 0.0f ? v : e;
                    } else {
                        elu = elu_fast16(v);  // the 16-bit paths' gate, as the fused kernel's
                    }
                    acc[j][k] = elu * g;
                }
        }
        if (valid && half == 0) {
#pragma unroll
            for (int j = 0; j < X; ++j) {
                const int ox = x0 + j;
                if (ox >= w) continue;
                T* po = at_mut<T>(dst, b, oy, ox, vidx * V);
                if (nv == V) {
                    if constexpr (sizeof(T) == 4) {
                        *reinterpret_cast<f32x4*>(po) = f32x4{acc[j][0], acc[j][1], acc[j][2], acc[j][3]};
                    } else {
                        typedef T t8 __attribute__((ext_vector_type(8)));
                        t8 hv;
#pragma unroll
                        for (int k = 0; k < 8; ++k) hv[k] = (T)acc[j][k];
                        *reinterpret_cast<t8*>(po) = hv;
                    }
                } else {
#pragma unroll
                    for (int k = 0; k < V; ++k)
                        if (k < nv) po[k] = from_f32<T>(acc[j][k]);
                }
            }
        }
#pragma unroll
        for (int j = 0; j < X + 2; ++j) {
            win[0][j] = win[1][j];
            win[1][j] = win[2][j];
        }
    }
}

// ------------------------------------------------------------------------------ layer norm
// `layer_norm_channels` (src/nn/fast/math.rs:423-448): f64 sums over channels in order,
// (x - mean) / sqrt(var + 1e-5) * w + b with f32 operations.
// A block stages LN_P positions x C channels in LDS with coalesced 16-byte loads (rows padded by
// one float against bank conflicts); one thread per position then sums its row in channel
// order, and all threads write the normalised values back coalesced.
template <typename T>
__global__ void __launch_bounds__(256) k_layer_norm(View src, View dst, int N, int C, int h, int w,
                                                    const float* wt, const float* bs, int P) {
    extern __shared__ float s_ln[];  // [P][C + 1], then mean[P], den[P]
    const int ld = C + 1, q = C / 4;
    float* s_m = s_ln + P * ld;
    float* s_d = s_m + P;
    const long long npos = (long long)N * h * w, p0 = (long long)blockIdx.x * P;
    for (int u = threadIdx.x; u < P * q; u += blockDim.x) {
        const int pl = u / q, cq = u - pl * q;
        f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
        if (p0 + pl < npos) {
            const Idx4 d = split(p0 + pl, h, w, 1);
            v = load4<T>(at<T>(src, d.b, d.y, d.x, cq * 4));
        }
        float* r = s_ln + pl * ld + cq * 4;
        r[0] = v[0]; r[1] = v[1]; r[2] = v[2]; r[3] = v[3];
    }
    __syncthreads();
    if ((int)threadIdx.x < P) {
        const float* r = s_ln + threadIdx.x * ld;
        double mean = 0.0;
        for (int c = 0; c < C; ++c) mean += (double)r[c];
        mean /= (double)C;
        double var = 0.0;
        for (int c = 0; c < C; ++c) { const double e = (double)r[c] - mean; var = var + e * e; }
        s_m[threadIdx.x] = (float)mean;
        s_d[threadIdx.x] = sqrtf((float)(var / (double)C) + 1e-5f);
    }
    __syncthreads();
    for (int u = threadIdx.x; u < P * q; u += blockDim.x) {
        const int pl = u / q, cq = u - pl * q;
        if (p0 + pl >= npos) continue;
        const Idx4 d = split(p0 + pl, h, w, 1);
        const float* r = s_ln + pl * ld + cq * 4;
        f32x4 o;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float e = r[k] - s_m[pl];
            e = e / s_d[pl];
            e = e * wt[cq * 4 + k];
            o[k] = e + bs[cq * 4 + k];
        }
        store4<T>(at_mut<T>(dst, d.b, d.y, d.x, cq * 4), o);
    }
}

// ------------------------------------------------------------------------ channel attention
// Per head h (c = dim / heads channels): S_ij = q_i . k_j, |q_i|^2 and |k_j|^2 summed over the
// n = h*w positions. One wave per head per chunk of ATT_POS positions runs the q . k sums on
// f32 MFMA (M = q channels, N = k channels, K = 4 positions per instruction) and the squared
// norms on f32 fma; the chunk partials are reduced in f64 by the softmax kernel.
constexpr int ATT_POS = 256;
int attention_gram_chunks(int h, int w) { return (h * w + ATT_POS - 1) / ATT_POS; }

// The chunk's q and k (the first 2 dim channels of qkv) pass through LDS, 32 KB of positions at
// a time (GRAM_SUB<T> = 32 f32 or 64 16-bit positions of 2 dim = 256 channels), as stored: every
// global load is a coalesced 16-byte read of a position's channel run, and the MFMA fragments
// are read from LDS and widened to f32 there. Wave w takes head h0 + w of each group of four heads
// (the synthesis nets have four: one group). The q . k sums run on MFMA in groups of 4 positions
// (a partial last group padded with zeros); |q_i|^2 and |k_j|^2 are f32 fmas in the lane that
// holds the element (lane l takes positions congruent to l / 16 mod 4), added across the four
// lane groups at the end. 35 KB of LDS per workgroup: four per CU overlap one another's loads
// and sums. An LDS row is 2 dim + 16 elements: at dim 128 the four position rows a wave reads
// fall on disjoint banks.
template <typename T>
constexpr int GRAM_SUB = 128 / (int)sizeof(T);
constexpr int GRAM_PAD = 16;

constexpr int GRAM_UNR = 8;
// Whether the staging takes fixed per-thread offsets (see the kernel): one round of loads per
// sub-chunk, dense positions, and 16-byte units per position dividing the workgroup.
template <typename T>
static bool gram_fast(const View& qkv, int dim, int w) {
    const int upp = 2 * dim / (16 / (int)sizeof(T));
    return upp > 0 && GRAM_SUB<T> * upp <= GRAM_UNR * 256 && qkv.row == (long long)w * qkv.cs && 256 % upp == 0;
}

template <typename T, bool FAST, int NB>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4)))
k_attention_gram(View qkv, int dim, int heads, int n, int w, float* partial) {
    extern __shared__ __align__(16) unsigned char s_raw[];
    T* s_qk = reinterpret_cast<T*>(s_raw);  // [GRAM_SUB][2 dim + GRAM_PAD]
    constexpr int VEC = 16 / (int)sizeof(T), SUB = GRAM_SUB<T>;
    const int c = dim / heads, E = c * c + 2 * c;  // NB = (c + 15) / 16 head blocks
    const int ld = 2 * dim + GRAM_PAD, upp = 2 * dim / VEC;  // LDS row; 16-byte units per position
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int m = lane & 15, kq = lane >> 4;
    const int b = blockIdx.y, nchunk = gridDim.x;
    const int p0 = blockIdx.x * ATT_POS;
    const int p1 = min(p0 + ATT_POS, n);
    const T* base = (const T*)qkv.p + (long long)b * qkv.bstride + qkv.c_off;
    const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
    // Staging: up to UNR 16-byte loads per thread in flight before the first wait. When a
    // sub-chunk is one round of them (units <= UNR * 256: dim <= 128), positions are dense
    // (row = w * cs) and upp divides 256, thread t's unit is t % upp of positions t / upp + k * pst
    // of the sub-chunk, k < UNR (pst = 256 / upp): fixed offsets, computed once.
    constexpr int UNR = GRAM_UNR;
    const int units = SUB * upp;
    constexpr bool fast = FAST;
    const int pst = fast ? 256 / upp : 0, fpl = fast ? threadIdx.x / upp : 0;
    const int fq = threadIdx.x - fpl * upp;
    const int fg = fpl * qkv.cs + fq * VEC, fs = fpl * ld + fq * VEC;
    // Fast path: the next sub-chunk's loads go out before this one's sums, so they fly meanwhile.
    u32x4 raw[UNR];
    auto fetch = [&](int ps) __attribute__((always_inline)) {
        const T* bp = base + (long long)ps * qkv.cs + fg;
        const int np = min(ps + SUB, p1) - ps;
#pragma unroll
        for (int k = 0; k < UNR; ++k) {
            raw[k] = u32x4{0u, 0u, 0u, 0u};
            if (fpl + k * pst < np) raw[k] = *(const u32x4*)(bp + k * pst * qkv.cs);
        }
    };
    for (int h0 = 0; h0 < heads; h0 += 4) {
        const int hd = h0 + wave;  // a wave past the last head only stages
        f32x4 g[2][2] = {{z, z}, {z, z}};
        float sq[2] = {0.0f, 0.0f}, sk[2] = {0.0f, 0.0f};
        if constexpr (FAST) fetch(p0);
        for (int ps = p0; ps < p1; ps += SUB) {
            const int pe = min(ps + SUB, p1);
            __syncthreads();  // the previous sub-chunk's reads are done
            if constexpr (FAST) {
#pragma unroll
                for (int k = 0; k < UNR; ++k)
                    if (fpl + k * pst < SUB) *reinterpret_cast<u32x4*>(s_qk + fs + k * pst * ld) = raw[k];
            } else {
                for (int u0 = threadIdx.x; u0 < units; u0 += UNR * 256) {
                    u32x4 raw[UNR];
#pragma unroll
                    for (int k = 0; k < UNR; ++k) {
                        const int u = u0 + k * 256;
                        const int pl = u / upp, pos = ps + pl;
                        raw[k] = u32x4{0u, 0u, 0u, 0u};
                        if (u < units && pos < pe) {
                            const int y = pos / w, x = pos - y * w, q = u - pl * upp;
                            raw[k] = *(const u32x4*)(base + (long long)y * qkv.row + (long long)x * qkv.cs + q * VEC);
                        }
                    }
#pragma unroll
                    for (int k = 0; k < UNR; ++k) {
                        const int u = u0 + k * 256;
                        if (u >= units) break;
                        const int pl = u / upp, q = u - pl * upp;
                        *reinterpret_cast<u32x4*>(s_qk + pl * ld + q * VEC) = raw[k];
                    }
                }
            }
            __syncthreads();
            if constexpr (FAST)
                if (ps + SUB < p1) fetch(ps + SUB);
            if (hd >= heads) continue;  // uniform per wave
            // Every LDS read is unconditional (row clamped into the sub-chunk; the element of a
            // position past pe or a channel past the head is then replaced by 0), so a group's
            // reads issue together instead of each waiting in its own branch.
            for (int p = ps; p < pe; p += 4) {
                float aq[NB], ak[NB];
                const T* r = s_qk + min(p - ps + kq, SUB - 1) * ld + hd * c + m;
                const bool ok = p + kq < pe;
#pragma unroll
                for (int bb = 0; bb < NB; ++bb) {
                    const bool in = ok && bb * 16 + m < c;
                    const float vq = (float)r[bb * 16], vk = (float)r[dim + bb * 16];
                    aq[bb] = in ? vq : 0.0f;
                    ak[bb] = in ? vk : 0.0f;
                    sq[bb] = fmaf(aq[bb], aq[bb], sq[bb]);
                    sk[bb] = fmaf(ak[bb], ak[bb], sk[bb]);
                }
#pragma unroll
                for (int bi = 0; bi < NB; ++bi)
#pragma unroll
                    for (int bj = 0; bj < NB; ++bj)
                        g[bi][bj] = __builtin_amdgcn_mfma_f32_16x16x4f32(aq[bi], ak[bj], g[bi][bj], 0, 0, 0);
            }
        }
        if (hd >= heads) continue;
#pragma unroll
        for (int bb = 0; bb < 2; ++bb) {
            sq[bb] += __shfl_xor(sq[bb], 16);
            sq[bb] += __shfl_xor(sq[bb], 32);
            sk[bb] += __shfl_xor(sk[bb], 16);
            sk[bb] += __shfl_xor(sk[bb], 32);
        }
        // Lane l holds D[4 * (l / 16) + i][l % 16] of each 16x16 tile.
        float* out = partial + (((long long)b * nchunk + blockIdx.x) * heads + hd) * E;
#pragma unroll
        for (int bi = 0; bi < 2; ++bi) {
            if (bi >= NB) continue;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = 4 * kq + i;
                if (bi * 16 + r >= c) continue;
#pragma unroll
                for (int bj = 0; bj < 2; ++bj)
                    if (bj < NB && bj * 16 + m < c) out[(bi * 16 + r) * c + bj * 16 + m] = g[bi][bj][i];
            }
            if (kq == 0 && bi * 16 + m < c) {
                out[c * c + bi * 16 + m] = sq[bi];
                out[c * c + c + bi * 16 + m] = sk[bi];
            }
        }
    }
}

// One workgroup per attention row (item b, head hd, query i): reduce the chunk partials in f64
// (in the fixed slice order described below, not position order), then divide the raw q . k
// dot by max(|q|, 1e-12) * max(|k|, 1e-12) -- the reference normalises q and k before the dot
// (F.normalize, src/nn/fast/math.rs:538-545), so the two agree to rounding, not bit for bit --,
// scale by the temperature and take the softmax with the Cephes exp and an f64 sum in index
// order (math.rs:558-577).
__global__ void __launch_bounds__(256) k_attention_softmax(const float* partial, int nchunk, int dim,
                                                           int heads, const float* temperature,
                                                           float* attn) {
    // The chunk sums run in ATT_SL slices of 32 lanes (slice t takes chunks t, t + ATT_SL, ...,
    // in order), then the slices are added in slice order: a fixed order, so the result does not
    // depend on scheduling, and ATT_SL times the loads in flight of a single 32-lane pass.
    constexpr int ATT_SL = 8;
    __shared__ double s_red[ATT_SL][2][32];
    __shared__ double s_rq[ATT_SL];
    __shared__ double s_qq;
    __shared__ float s_e[64];
    const int row = blockIdx.x, b = blockIdx.y, c = dim / heads, hd = row / c, i = row - hd * c;
    const int E = c * c + 2 * c, tid = threadIdx.x, sl = tid >> 5, j = tid & 31;
    // Every lane of a row also sums |q_i|^2 (the same address across the row, so the loads of an
    // iteration carry no branch and successive iterations' loads overlap); lane 0's sum is used.
    double sqk = 0.0, skk = 0.0, sqq = 0.0;
    if (j < c) {
#pragma unroll 4
        for (int k = sl; k < nchunk; k += ATT_SL) {
            const float* pb = partial + (((long long)b * nchunk + k) * heads + hd) * E;
            const float vqk = pb[i * c + j], vkk = pb[c * c + c + j], vqq = pb[c * c + i];
            sqk += (double)vqk;
            skk += (double)vkk;
            sqq += (double)vqq;
        }
    }
    s_red[sl][0][j] = sqk;
    s_red[sl][1][j] = skk;
    if (j == 0) s_rq[sl] = sqq;
    __syncthreads();
    const int lane = tid;  // the rest runs on threads 0..63 (columns j < c)
    sqk = 0.0;
    skk = 0.0;
    if (lane < c) {
        for (int t = 0; t < ATT_SL; ++t) {
            sqk += s_red[t][0][lane];
            skk += s_red[t][1][lane];
        }
    }
    if (lane == 0) {
        double q = 0.0;
        for (int t = 0; t < ATT_SL; ++t) q += s_rq[t];
        s_qq = q;
    }
    __syncthreads();
    float nq = (float)sqrt(s_qq);
    nq = nq > 1e-12f ? nq : 1e-12f;
    float a = -INFINITY;
    if (lane < c) {
        float nk = (float)sqrt(skk);
        nk = nk > 1e-12f ? nk : 1e-12f;
        a = (float)(sqk / ((double)nq * (double)nk)) * temperature[hd];
    }
    if (lane < 64) s_e[lane] = a;
    __syncthreads();
    float mx = -INFINITY;
    for (int jj = 0; jj < c; ++jj) mx = fmaxf(mx, s_e[jj]);
    __syncthreads();
    if (lane < c) s_e[lane] = cephes_exp(a - mx);
    __syncthreads();
    double sum = 0.0;
    for (int jj = 0; jj < c; ++jj) sum += (double)s_e[jj];
    if (lane < c) attn[((long long)b * dim + row) * c + lane] = s_e[lane] / (float)sum;
}

// Folds the output projection into the attention: wfold[o][hd*c + j] =
// sum_i proj[o][hd*c + i] * attn[hd*c + i][j] (f64 accumulate), stored straight into the packed
// 1x1 conv layout [chunk][nblk][16][CK] of the storage type, one weight per batch item. A null
// proj is the identity (the same products, 1 or 0 times attn).
template <typename T>
__global__ void k_attention_fold(const float* proj, const float* attn, int dim, int heads, int nblk,
                                 int CK, T* wpk, long long w_bstride) {
    const int e = blockIdx.x * blockDim.x + threadIdx.x, b = blockIdx.y;
    if (e >= dim * dim) return;
    const int c = dim / heads, o = e / dim, col = e - o * dim, hd = col / c, j = col - hd * c;
    const float* at_b = attn + (long long)b * dim * c;
    // All c (<= 32) operand pairs are loaded before the first product (indices clamped to the
    // head), so the loads overlap instead of each waiting for the previous one's sum.
    float pw[32], av[32];
    if (proj) {
#pragma unroll
        for (int i = 0; i < 32; ++i) pw[i] = proj[o * dim + hd * c + min(i, c - 1)];
    } else {
#pragma unroll
        for (int i = 0; i < 32; ++i) pw[i] = o == hd * c + min(i, c - 1) ? 1.0f : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < 32; ++i) av[i] = at_b[(hd * c + min(i, c - 1)) * c + j];
    double s = 0.0;
#pragma unroll
    for (int i = 0; i < 32; ++i)
        if (i < c) s += (double)pw[i] * (double)av[i];
    const int ch = col / CK, kk = col - ch * CK;
    wpk[(long long)b * w_bstride + (((long long)ch * nblk + o / 16) * 16 + o % 16) * CK + kk] = from_f32<T>((float)s);
}

// Zero fill with vector stores (instead of hipMemsetAsync, which callers capturing the stream
// into a HIP graph cannot rely on): n 4-byte words, then `tail` (< 4) bytes after them.
__global__ void k_zero_u32(uint32_t* p, long long n, int tail) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        p[i] = 0u;
    } else if (i == n) {
        unsigned char* t = reinterpret_cast<unsigned char*>(p + n);
        for (int k = 0; k < tail; ++k) t[k] = 0;
    }
}

// Non-finite f16 samples (exponent field all ones: +-inf from an overflow past 65504, or NaN) of
// an N x [h][w][C] view, added to slots[blockIdx.x]. A fixed grid of `nslots` workgroups walks
// the view; each workgroup sums its count in LDS and one thread adds it to its own slot, so no
// two workgroups write one slot and successive launches on one stream accumulate in order.
__global__ void __launch_bounds__(256) k_count_f16_nonfinite(View v, int N, int C, int h, int w,
                                                             unsigned long long* slots) {
    __shared__ unsigned int s_cnt[256];
    const long long total = (long long)N * h * w * C;
    const uint16_t* base = reinterpret_cast<const uint16_t*>(v.p);
    unsigned int cnt = 0;
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < total; i += (long long)gridDim.x * 256) {
        const int c = (int)(i % C);
        long long r = i / C;
        const int x = (int)(r % w);
        r /= w;
        const int y = (int)(r % h);
        const int b = (int)(r / h);
        const uint16_t bits = base[(long long)b * v.bstride + (long long)y * v.row + (long long)x * v.cs + v.c_off + c];
        cnt += (bits & 0x7c00u) == 0x7c00u ? 1u : 0u;
    }
    s_cnt[threadIdx.x] = cnt;
    __syncthreads();
    for (int k = 128; k > 0; k >>= 1) {
        if ((int)threadIdx.x < k) s_cnt[threadIdx.x] += s_cnt[threadIdx.x + k];
        __syncthreads();
    }
    if (threadIdx.x == 0 && s_cnt[0]) slots[blockIdx.x] += s_cnt[0];
}

// ------------------------------------------------------------------------------- launchers
static inline dim3 grid_for(long long n) { return dim3((unsigned)((n + 255) / 256)); }

hipError_t launch_count_f16_nonfinite(View v, int N, int C, int h, int w, unsigned long long* slots,
                                      int nslots, hipStream_t s) {
    if (N <= 0 || C <= 0 || h <= 0 || w <= 0 || nslots <= 0) return hipSuccess;
    k_count_f16_nonfinite<<<dim3((unsigned)nslots), 256, 0, s>>>(v, N, C, h, w, slots);
    return hipGetLastError();
}

hipError_t launch_zero(void* p, size_t bytes, hipStream_t s) {
    if ((uintptr_t)p & 3) return hipErrorInvalidValue;
    const long long n = (long long)(bytes / 4);
    const int tail = (int)(bytes % 4);
    if (bytes == 0) return hipSuccess;
    k_zero_u32<<<grid_for(n + (tail ? 1 : 0)), 256, 0, s>>>((uint32_t*)p, n, tail);
    return hipGetLastError();
}

#define ZJAI_DISPATCH(dtype, KERNEL, ...)                                                     \
    switch (dtype) {                                                                         \
        case DT_F32: KERNEL<float> __VA_ARGS__; break;                                       \
        case DT_F16: KERNEL<_Float16> __VA_ARGS__; break;                                    \
        case DT_BF16: KERNEL<__bf16> __VA_ARGS__; break;                                     \
        default: return hipErrorInvalidValue;                                                \
    }

hipError_t launch_planar_to_nhwc(const float* src, int C, int LH, int LW, const Windows& win, int N,
                                 int h, int w, View dst, int dtype, hipStream_t s) {
    if (C % 4 || N < 1 || N > MAXB) return hipErrorInvalidValue;
    for (int b = 0; b < N; ++b)
        if (win.y0[b] < 0 || win.x0[b] < 0 || win.y0[b] + h > LH || win.x0[b] + w > LW) return hipErrorInvalidValue;
    const long long n = (long long)N * h * ((w + PT_X - 1) / PT_X);
    if (n == 0 || C == 0) return hipSuccess;
    if (n > 0x7ffffff0LL) return hipErrorInvalidValue;
    const unsigned nb = (unsigned)((n + 7) / 8 * 8);
    ZJAI_DISPATCH(dtype, k_planar_to_nhwc, <<<dim3(nb), 256, 0, s>>>(src, C, LH, LW, win, N, h, w, dst))
    return hipGetLastError();
}

hipError_t launch_nhwc_to_planar(View src, int dtype, int N, int C, int h, int w, float* dst,
                                 hipStream_t s) {
    const long long n = (long long)N * h * w * ((C + 3) / 4);
    if (n == 0) return hipSuccess;
    ZJAI_DISPATCH(dtype, k_nhwc_to_planar, <<<grid_for(n), 256, 0, s>>>(src, N, C, h, w, dst))
    return hipGetLastError();
}

hipError_t launch_eltwise(int op, View x, View src, int dtype, int N, int C, int h, int w,
                          hipStream_t s) {
    const long long n = (long long)N * h * w * (C / 4);
    if (n == 0) return hipSuccess;
    ZJAI_DISPATCH(dtype, k_eltwise, <<<grid_for(n), 256, 0, s>>>(op, x, src, N, C, h, w))
    return hipGetLastError();
}

hipError_t launch_copy(View src, View dst, int dtype, int N, int C, int h, int w, hipStream_t s) {
    const long long n = (long long)N * h * w * (C / 4);
    if (n == 0) return hipSuccess;
    ZJAI_DISPATCH(dtype, k_copy, <<<grid_for(n), 256, 0, s>>>(src, dst, N, C, h, w))
    return hipGetLastError();
}

hipError_t launch_pixel_shuffle(View src, View dst, int dtype, int N, int C_out, int h, int w,
                                int r, hipStream_t s) {
    const long long n = (long long)N * h * r * w * r * (C_out / 4);
    if (n == 0) return hipSuccess;
    ZJAI_DISPATCH(dtype, k_pixel_shuffle, <<<grid_for(n), 256, 0, s>>>(src, dst, N, C_out, h, w, r))
    return hipGetLastError();
}

hipError_t launch_depthwise3x3(View src, View dst, int dtype, int N, int C, int h, int w,
                               const float* weight, const float* bias, int elu_half,
                               hipStream_t s) {
    const int cout = elu_half > 0 ? elu_half : C;
    if (cout % 4 || C % 4 || (elu_half > 0 && 2 * elu_half != C)) return hipErrorInvalidValue;
    const int V = dtype == DT_F32 ? 4 : 8, X = dtype == DT_F32 ? 4 : 2;  // Dw<T>
    const int vpw = elu_half > 0 ? 32 : 64;
    const long long waves = (long long)N * ((h + DW_R - 1) / DW_R) * ((w + X - 1) / X) *
                            (((cout + V - 1) / V + vpw - 1) / vpw);
    if (waves == 0) return hipSuccess;
    // a multiple of 8 workgroups for the kernel's XCD-aware block order (the extra ones exit)
    const long long blocks = ((waves + 3) / 4 + 7) / 8 * 8;
    if (blocks > (1ll << 31) - 1) return hipErrorInvalidValue;
    ZJAI_DISPATCH(dtype, k_depthwise3x3, <<<dim3((unsigned)blocks), 256, 0, s>>>(src, dst, N, C, h, w, weight, bias, elu_half))
    return hipGetLastError();
}

hipError_t launch_layer_norm(View src, View dst, int dtype, int N, int C, int h, int w,
                             const float* weight, const float* bias, hipStream_t s) {
    const long long n = (long long)N * h * w;
    if (n == 0) return hipSuccess;
    // Positions per block: as many as fit in 32 KiB of LDS, at most 64.
    const int P = std::max(1, std::min(64, 8192 / (C + 1)));
    const size_t lds = sizeof(float) * ((size_t)P * (C + 1) + 2 * P);
    if (lds > 64 * 1024) return hipErrorInvalidValue;
    const dim3 g((unsigned)((n + P - 1) / P));
    ZJAI_DISPATCH(dtype, k_layer_norm, <<<g, 256, lds, s>>>(src, dst, N, C, h, w, weight, bias, P))
    return hipGetLastError();
}

bool attention_gram_fits(int dtype, int dim) {
    if (dim <= 0) return false;
    const size_t lds = (size_t)(dtype == DT_F32 ? 4 * GRAM_SUB<float> : 2 * GRAM_SUB<__bf16>) * (2 * dim + GRAM_PAD);
    return lds <= 160 * 1024;
}

template <typename T>
static void gram_go(dim3 g, size_t lds, hipStream_t s, bool fast, int nb, View qkv, int dim, int heads, int n,
                    int w, float* partial) {
    if (fast) {
        if (nb == 1) k_attention_gram<T, true, 1><<<g, 256, lds, s>>>(qkv, dim, heads, n, w, partial);
        else k_attention_gram<T, true, 2><<<g, 256, lds, s>>>(qkv, dim, heads, n, w, partial);
    } else {
        if (nb == 1) k_attention_gram<T, false, 1><<<g, 256, lds, s>>>(qkv, dim, heads, n, w, partial);
        else k_attention_gram<T, false, 2><<<g, 256, lds, s>>>(qkv, dim, heads, n, w, partial);
    }
}

std::string attention_gram_name(const View& qkv, int dtype, int dim, int heads, int w) {
    static const char* ty[] = {"float", "_Float16", "__bf16"};
    if (dtype < DT_F32 || dtype > DT_BF16 || heads <= 0) return "k_attention_gram";
    const bool f = dtype == DT_F32 ? gram_fast<float>(qkv, dim, w)
                                   : dtype == DT_F16 ? gram_fast<_Float16>(qkv, dim, w) : gram_fast<__bf16>(qkv, dim, w);
    return std::string("k_attention_gram<") + ty[dtype] + (f ? ", true, " : ", false, ") +
           (dim / heads > 16 ? "2>" : "1>");
}

hipError_t launch_attention_gram(View qkv, int dtype, int N, int dim, int heads, int h, int w,
                                 float* partial, hipStream_t s) {
    const int c = heads > 0 ? dim / heads : 0;
    const int vec = dtype == DT_F32 ? 4 : 8;
    if (heads <= 0 || dim % heads || c < 1 || c > 32 || (2 * dim) % vec || qkv.cs % vec ||
        qkv.c_off % vec || qkv.row % vec || qkv.bstride % vec || (uintptr_t)qkv.p % 16)
        return hipErrorInvalidValue;
    const int nchunk = attention_gram_chunks(h, w);
    if (nchunk == 0 || N == 0) return hipSuccess;
    if (!attention_gram_fits(dtype, dim)) return hipErrorInvalidValue;
    const size_t lds = (size_t)(dtype == DT_F32 ? 4 * GRAM_SUB<float> : 2 * GRAM_SUB<__bf16>) * (2 * dim + GRAM_PAD);
    const dim3 g(nchunk, N);
    const int nb = (c + 15) / 16;
    switch (dtype) {
        case DT_F32: gram_go<float>(g, lds, s, gram_fast<float>(qkv, dim, w), nb, qkv, dim, heads, h * w, w, partial); break;
        case DT_F16: gram_go<_Float16>(g, lds, s, gram_fast<_Float16>(qkv, dim, w), nb, qkv, dim, heads, h * w, w, partial); break;
        case DT_BF16: gram_go<__bf16>(g, lds, s, gram_fast<__bf16>(qkv, dim, w), nb, qkv, dim, heads, h * w, w, partial); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_attention_softmax(const float* partial, int N, int nchunk, int dim, int heads,
                                    const float* temperature, float* attn, hipStream_t s) {
    if (heads <= 0 || dim % heads || dim / heads > 32) return hipErrorInvalidValue;
    k_attention_softmax<<<dim3(dim, N), 256, 0, s>>>(partial, nchunk, dim, heads, temperature, attn);
    return hipGetLastError();
}

hipError_t launch_attention_fold(const float* proj, const float* attn, int N, int dim, int heads,
                                 int dtype, int nblk, void* wpk, long long w_bstride,
                                 hipStream_t s) {
    if (heads <= 0 || dim % heads || dim / heads > 32) return hipErrorInvalidValue;  // k_attention_fold's c <= 32
    const int CK = dtype == DT_F32 ? 16 : 32;
    const dim3 g((dim * dim + 255) / 256, N);
    switch (dtype) {
        case DT_F32: k_attention_fold<float><<<g, 256, 0, s>>>(proj, attn, dim, heads, nblk, CK, (float*)wpk, w_bstride); break;
        case DT_F16: k_attention_fold<_Float16><<<g, 256, 0, s>>>(proj, attn, dim, heads, nblk, CK, (_Float16*)wpk, w_bstride); break;
        case DT_BF16: k_attention_fold<__bf16><<<g, 256, 0, s>>>(proj, attn, dim, heads, nblk, CK, (__bf16*)wpk, w_bstride); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace zjai
