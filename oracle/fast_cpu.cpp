// CPU baseline for the JPEG AI synthesis hot path. TEST INFRASTRUCTURE ONLY.
//
// A C++ restatement of the reference's CPU convolution engine, `nn::fast` (src/nn/fast/conv.rs),
// used as the `cpu_baseline` leg of bench.py (timed on the GPU box's host cores next to the HIP
// path) and pinned by tests to the oracle loops in oracle.cpp. The reference itself is Rust and
// cannot be built here, so its algorithm is restated rather than run:
//
//   * activations in channel-blocked NCHWc layout, [ceil(C/V)][H][W][V] (tensor.rs:1-5);
//   * weights packed once as [out block][in block][V in][tap][V out], zero beyond the real
//     channel counts (`pack`, conv.rs:457-488);
//   * per output row, the input strip is im2col-packed into [in block][tap][ow][V] and every
//     output block reads it at unit stride (`forward_blis`, conv.rs:1093-1237);
//   * the micro-kernel keeps B output positions x V output channels in registers and, per input
//     block, input channel and tap, broadcasts one input sample and adds weight-vector x sample
//     with a fused multiply-add (`block` / `tap_loop_n`, conv.rs:187-330); a row's tail is one
//     overlapping block (`conv_row_s`, conv.rs:340-377);
//   * a stride-2 transposed convolution runs per output row and column parity as a small
//     ordinary convolution over the input padded by 2 (`PackedConvTranspose`, conv.rs:1891-2028);
//   * rows are distributed over threads (rayon there, OpenMP here).
// Accumulation order per output is bias, then input channel ascending, then tap (ky, kx)
// ascending -- the order of `nn::reference` -- so every result equals the oracle bit for bit.
// Tiers as in the reference: AVX-512 V = 16, B = 24 (conv.rs:381-386); AVX2 V = 8, B = 12
// (conv.rs:388-393), chosen at run time.
//
// Grouped convolutions whose group size is not a multiple of V are not packed by the reference
// either (they go to its fallback kernel); here they run the oracle loops (or_conv2d), which have
// the same result. Depthwise layers run a row-vectorised kernel with the oracle's sum order.

#include <immintrin.h>
#include <omp.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <memory>
#include <vector>

extern "C" int or_conv2d(const float* x, int c, int h, int w, const float* weight, const float* bias,
                         int out_ch, int kh, int kw, int stride, int pad_h, int pad_w, int groups,
                         const int* extra, float* y);

namespace {

constexpr int MAXT = 9;

template <int V> struct Simd;
template <> struct Simd<16> {
    using T = __m512;
    __attribute__((target("avx512f"))) static T load(const float* p) { return _mm512_loadu_ps(p); }
    __attribute__((target("avx512f"))) static void store(float* p, T v) { _mm512_storeu_ps(p, v); }
    __attribute__((target("avx512f"))) static T splat(float x) { return _mm512_set1_ps(x); }
    __attribute__((target("avx512f"))) static T fma(T a, T b, T c) { return _mm512_fmadd_ps(a, b, c); }
};
template <> struct Simd<8> {
    using T = __m256;
    __attribute__((target("avx2,fma"))) static T load(const float* p) { return _mm256_loadu_ps(p); }
    __attribute__((target("avx2,fma"))) static void store(float* p, T v) { _mm256_storeu_ps(p, v); }
    __attribute__((target("avx2,fma"))) static T splat(float x) { return _mm256_set1_ps(x); }
    __attribute__((target("avx2,fma"))) static T fma(T a, T b, T c) { return _mm256_fmadd_ps(a, b, c); }
};

// One pass over an output row of one output block.
struct Row {
    float* out;        // output row, [ow][V]; writes positions o0 + j * os, j < n
    int o0, os, n;
    const float* x;    // strip: tap t of input block b at x + (b * xb + t * xt), position j at j*V*is
    long xb, xt;
    int is;            // input position step per output (1: im2col strip; 2: none here)
    int nb, in_ch;     // input blocks, real input channels
    int nt;            // taps
    const float* w;    // [nb][V][nt][V]
    const float* bias; // V
};

// B positions starting at output j: acc = bias; for in block, channel v < vin, tap:
// acc[b] = fma(w[v][t], x[t][j + b][v], acc[b]).
#define FC_INLINE __attribute__((always_inline)) inline

template <int V, int B, int NT>
FC_INLINE void block(const Row& r, int j) {
    using S = Simd<V>;
    typename S::T acc[B];
    const typename S::T b0 = S::load(r.bias);
    for (int b = 0; b < B; ++b) acc[b] = b0;
    const int nt = NT > 0 ? NT : r.nt;
    for (int ib = 0; ib < r.nb; ++ib) {
        const int vin = std::min(V, r.in_ch - ib * V);
        const float* wb = r.w + (long)ib * V * nt * V;
        const float* xb = r.x + ib * r.xb + (long)j * r.is * V;
        for (int v = 0; v < vin; ++v)
            for (int t = 0; t < nt; ++t) {
                const typename S::T wv = S::load(wb + ((long)v * nt + t) * V);
                const float* xs = xb + t * r.xt + v;
                for (int b = 0; b < B; ++b) acc[b] = S::fma(wv, S::splat(xs[(long)b * r.is * V]), acc[b]);
            }
    }
    for (int b = 0; b < B; ++b) S::store(r.out + (long)(r.o0 + (j + b) * r.os) * V, acc[b]);
}

template <int V, int B, int NT>
FC_INLINE void row_nt(const Row& r) {
    int j = 0;
    while (j + B <= r.n) {
        block<V, B, NT>(r, j);
        j += B;
    }
    if (j < r.n && r.n >= B) {  // one overlapping block covers the tail
        block<V, B, NT>(r, r.n - B);
        return;
    }
    for (; j + 8 <= r.n; j += 8) block<V, 8, NT>(r, j);
    for (; j + 4 <= r.n; j += 4) block<V, 4, NT>(r, j);
    for (; j < r.n; ++j) block<V, 1, NT>(r, j);
}

template <int V, int B>
FC_INLINE void run_row(const Row& r) {
    switch (r.nt) {
        case 1: row_nt<V, B, 1>(r); break;
        case 4: row_nt<V, B, 4>(r); break;
        case 9: row_nt<V, B, 9>(r); break;
        default: row_nt<V, B, 0>(r); break;
    }
}

__attribute__((target("avx512f"))) void run_row16(const Row& r) { run_row<16, 24>(r); }
__attribute__((target("avx2,fma"))) void run_row8(const Row& r) { run_row<8, 12>(r); }

int g_forced_v = 0;  // fc_force_tier (tests run both tiers)

int tier_v() {
    static const int v = __builtin_cpu_supports("avx512f") ? 16 : 8;
    return g_forced_v ? g_forced_v : v;
}

void dispatch(int V, const Row& r) {
    if (V == 16) run_row16(r);
    else run_row8(r);
}

// An uninitialised float buffer (every element is written before it is read).
struct FBuf {
    std::unique_ptr<float[]> p;
    explicit FBuf(size_t n) : p(new float[n]) {}
    float* data() { return p.get(); }
    const float* data() const { return p.get(); }
};

// planar [c][h][w] -> NCHWc [ceil(c/V)][h][w][V] with left/top/right/bottom zero borders. One
// (block, padded row) per iteration: V contiguous source rows into one contiguous destination
// row, so no cache line is fetched more than once.
FBuf to_blocked(const float* x, int c, int h, int w, int V, int pt, int pl, int pb, int pr) {
    const int nb = (c + V - 1) / V, ph = h + pt + pb, pw = w + pl + pr;
    FBuf o((size_t)nb * ph * pw * V);
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < nb; ++b)
        for (int r = 0; r < ph; ++r) {
            float* d = o.data() + ((size_t)b * ph + r) * pw * V;
            const int yy = r - pt;
            if (yy < 0 || yy >= h) {
                std::memset(d, 0, sizeof(float) * pw * V);
                continue;
            }
            std::memset(d, 0, sizeof(float) * pl * V);
            std::memset(d + (size_t)(pl + w) * V, 0, sizeof(float) * pr * V);
            for (int v = 0; v < V; ++v) {
                const int ch = b * V + v;
                float* dv = d + (size_t)pl * V + v;
                if (ch >= c) {
                    for (int xx = 0; xx < w; ++xx) dv[(size_t)xx * V] = 0.0f;
                    continue;
                }
                const float* s = x + ((size_t)ch * h + yy) * w;
                for (int xx = 0; xx < w; ++xx) dv[(size_t)xx * V] = s[xx];
            }
        }
    return o;
}

// NCHWc -> planar, one (block, row) per iteration as in to_blocked.
void from_blocked(const float* o, int c, int h, int w, int V, float* y) {
    const int nb = (c + V - 1) / V;
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < nb; ++b)
        for (int yy = 0; yy < h; ++yy) {
            const float* s = o + ((size_t)b * h + yy) * w * V;
            for (int v = 0; v < V && b * V + v < c; ++v) {
                float* d = y + ((size_t)(b * V + v) * h + yy) * w;
                for (int xx = 0; xx < w; ++xx) d[xx] = s[(size_t)xx * V + v];
            }
        }
}

// [oc][ic][t] accessor -> [ocb][icb][V in][t][V out].
template <typename F>
std::vector<float> pack(int V, int out_ch, int in_ch, int nt, F get) {
    const int ocb = (out_ch + V - 1) / V, icb = (in_ch + V - 1) / V;
    std::vector<float> w((size_t)ocb * icb * V * nt * V, 0.0f);
#pragma omp parallel for schedule(static)
    for (int oc = 0; oc < out_ch; ++oc)
        for (int ic = 0; ic < in_ch; ++ic)
            for (int t = 0; t < nt; ++t)
                w[((((size_t)(oc / V) * icb + ic / V) * V + ic % V) * nt + t) * V + oc % V] = get(oc, ic, t);
    return w;
}

std::vector<float> pack_bias(int V, int out_ch, const float* bias) {
    std::vector<float> b((size_t)((out_ch + V - 1) / V) * V, 0.0f);
    if (bias) std::memcpy(b.data(), bias, sizeof(float) * out_ch);
    return b;
}

}  // namespace

extern "C" {

// The tier's block size (16 with AVX-512, else 8).
int fc_block_size(void) { return tier_v(); }

// Threads the OpenMP loops use.
int fc_threads(void) { return omp_get_max_threads(); }

// Sets the threads of later OpenMP loops (this library's and oracle.cpp's); n >= 1.
int fc_set_threads(int n) {
    if (n < 1) return -1;
    omp_set_num_threads(n);
    return 0;
}

// Forces the AVX2 tier (v = 8), the AVX-512 tier (16, only where supported) or automatic (0).
int fc_force_tier(int v) {
    if (v != 0 && v != 8 && !(v == 16 && __builtin_cpu_supports("avx512f"))) return -1;
    g_forced_v = v;
    return 0;
}

// Depthwise convolution (one input and one output channel per group, stride 1), planar: per
// channel the zero-padded plane, then per tap (ky, kx ascending) one fused multiply-add over a
// whole output row -- per output bias, then the taps in order, the oracle's sum -- vectorised
// along the row by the compiler; OpenMP over channels (the reference's depthwise kernel,
// src/nn/fast/depthwise.rs, likewise walks rows of one channel).
static int depthwise(const float* x, int c, int h, int w, const float* weight, const float* bias, int kh,
                     int kw, int pt, int pl, int pb, int pr, float* y) {
    const int ph = h + pt + pb, pw = w + pl + pr;
    if (ph < kh || pw < kw) return -1;
    const int oh = ph - kh + 1, ow = pw - kw + 1;
#pragma omp parallel
    {
        std::vector<float> pad((size_t)ph * pw);
#pragma omp for schedule(dynamic, 1)
        for (int ch = 0; ch < c; ++ch) {
            std::fill(pad.begin(), pad.end(), 0.0f);
            for (int r = 0; r < h; ++r)
                std::memcpy(pad.data() + (size_t)(r + pt) * pw + pl, x + ((size_t)ch * h + r) * w, sizeof(float) * w);
            const float* k = weight + (size_t)ch * kh * kw;
            const float b = bias ? bias[ch] : 0.0f;
            for (int oy = 0; oy < oh; ++oy) {
                float* o = y + ((size_t)ch * oh + oy) * ow;
                for (int ox = 0; ox < ow; ++ox) o[ox] = b;
                for (int ky = 0; ky < kh; ++ky)
                    for (int kx = 0; kx < kw; ++kx) {
                        const float wt = k[ky * kw + kx];
                        const float* in = pad.data() + (size_t)(oy + ky) * pw + kx;
                        for (int ox = 0; ox < ow; ++ox) o[ox] = std::fma(wt, in[ox], o[ox]);
                    }
            }
        }
    }
    return 0;
}

// Convolution, planar in / planar out, the same arguments and result as or_conv2d.
int fc_conv2d(const float* x, int c, int h, int w, const float* weight, const float* bias, int out_ch,
              int kh, int kw, int stride, int pad_h, int pad_w, int groups, const int* extra, float* y) {
    const int V = tier_v();
    if (groups <= 0 || c % groups || out_ch % groups || stride <= 0 || kh <= 0 || kw <= 0) return -1;
    const int icg = c / groups, ocg = out_ch / groups, nt = kh * kw;
    if (groups == c && groups == out_ch && stride == 1)
        return depthwise(x, c, h, w, weight, bias, kh, kw, pad_h + (extra ? extra[0] : 0), pad_w + (extra ? extra[1] : 0),
                         pad_h + (extra ? extra[2] : 0), pad_w + (extra ? extra[3] : 0), y);
    if (nt > MAXT || stride > 2 || (groups > 1 && (icg % V || ocg % V)))
        return or_conv2d(x, c, h, w, weight, bias, out_ch, kh, kw, stride, pad_h, pad_w, groups, extra, y);
    const int pt = pad_h + (extra ? extra[0] : 0), pl = pad_w + (extra ? extra[1] : 0);
    const int pb = pad_h + (extra ? extra[2] : 0), pr = pad_w + (extra ? extra[3] : 0);
    const int ph = h + pt + pb, pw = w + pl + pr;
    if (ph < kh || pw < kw) return -1;
    const int oh = (ph - kh) / stride + 1, ow = (pw - kw) / stride + 1;
    const FBuf xb = to_blocked(x, c, h, w, V, pt, pl, pb, pr);
    // Per group, packed weights [ocb][icb][V][nt][V] and bias.
    std::vector<std::vector<float>> wp(groups);
    for (int g = 0; g < groups; ++g)
        wp[g] = pack(V, ocg, icg, nt, [&](int oc, int ic, int t) {
            return weight[((size_t)(g * ocg + oc) * icg + ic) * nt + t];
        });
    const std::vector<float> bp = pack_bias(V, out_ch, bias);
    const int icbg = (icg + V - 1) / V, ocbg = (ocg + V - 1) / V, ocb = (out_ch + V - 1) / V;
    FBuf yb((size_t)ocb * oh * ow * V);
    const long wlen = (long)icbg * V * nt * V;
#pragma omp parallel
    {
        std::vector<float> strip((size_t)icbg * nt * ow * V);
#pragma omp for schedule(dynamic, 1)
        for (int oy = 0; oy < oh * groups; ++oy) {
            const int g = oy / oh, r = oy % oh;
            // im2col strip of this row and group: [icb][tap][ow][V].
            for (int ib = 0; ib < icbg; ++ib) {
                const float* xs = xb.data() + (size_t)(g * icbg + ib) * ph * pw * V;
                for (int ky = 0; ky < kh; ++ky)
                    for (int kx = 0; kx < kw; ++kx) {
                        float* d = strip.data() + ((size_t)(ib * nt + ky * kw + kx) * ow) * V;
                        const float* s = xs + ((size_t)(r * stride + ky) * pw + kx) * V;
                        for (int m = 0; m < ow; ++m) std::memcpy(d + (size_t)m * V, s + (size_t)m * stride * V, sizeof(float) * V);
                    }
            }
            for (int ob = 0; ob < ocbg; ++ob) {
                const int gob = g * ocbg + ob;
                Row rw{yb.data() + ((size_t)gob * oh + r) * ow * V, 0, 1, ow,
                       strip.data(), (long)nt * ow * V, (long)ow * V, 1, icbg, icg, nt,
                       wp[g].data() + ob * wlen, bp.data() + (size_t)gob * V};
                dispatch(V, rw);
            }
        }
    }
    from_blocked(yb.data(), out_ch, oh, ow, V, y);
    return 0;
}

// Stride-2 transposed convolution (k <= 4), planar in / out, as or_conv_transpose2d.
int fc_conv_transpose2d(const float* x, int c, int h, int w, const float* weight, const float* bias,
                        int out_ch, int k, int stride, int pad, int out_pad, float* y) {
    const int V = tier_v();
    if (stride != 2 || k > 4 || pad >= k || out_pad >= stride || h <= 0 || w <= 0) return -1;
    const int EXT = 2;
    const int oh = (h - 1) * 2 + k + out_pad - 2 * pad, ow = (w - 1) * 2 + k + out_pad - 2 * pad;
    const int ph = h + 2 * EXT, pw = w + 2 * EXT;
    const FBuf xb = to_blocked(x, c, h, w, V, EXT, EXT, EXT, EXT);
    // Phase (row parity a, column parity b) of ky / kx: the taps with ky % 2 == a, kx % 2 == b,
    // ascending, (ky, kx) order; weights [in][out][k][k].
    std::vector<int> kys[2], kxs[2];
    for (int p = 0; p < 2; ++p)
        for (int kk = 0; kk < k; ++kk)
            if (kk % 2 == p) kys[p].push_back(kk), kxs[p].push_back(kk);
    std::vector<float> wph[2][2];
    for (int a = 0; a < 2; ++a)
        for (int b = 0; b < 2; ++b) {
            const int nx = (int)kxs[b].size(), nt = (int)kys[a].size() * nx;
            if (!nt) continue;
            wph[a][b] = pack(V, out_ch, c, nt, [&](int oc, int ic, int t) {
                const int ky = kys[a][t / nx], kx = kxs[b][t % nx];
                return weight[(((size_t)ic * out_ch + oc) * k + ky) * k + kx];
            });
        }
    const std::vector<float> bp = pack_bias(V, out_ch, bias);
    const int icb = (c + V - 1) / V, ocb = (out_ch + V - 1) / V;
    FBuf yb((size_t)ocb * oh * ow * V);
#pragma omp parallel
    {
        // Per tap, the input row read by this output row, gathered as a strip [icb][tap][n][V].
        std::vector<float> strip((size_t)icb * 4 * (ow / 2 + 2) * V);
#pragma omp for schedule(dynamic, 1)
        for (int oy = 0; oy < oh; ++oy) {
            const int a = (oy + pad) % 2;
            for (int q = 0; q < std::min(2, ow); ++q) {
                const int b = (q + pad) % 2;
                const int nx = (int)kxs[b].size(), nt = (int)kys[a].size() * nx;
                const int n = (ow - q + 1) / 2;
                for (int ib = 0; ib < icb; ++ib) {
                    const float* xs = xb.data() + (size_t)ib * ph * pw * V;
                    for (int t = 0; t < nt; ++t) {
                        const int ky = kys[a][t / nx], kx = kxs[b][t % nx];
                        // floor((oy + pad - ky) / 2) + EXT, likewise for the column of output q.
                        const int iy = (oy + pad - ky + 2 * EXT) / 2;
                        const int ix = (q + pad - kx + 2 * EXT) / 2;
                        float* d = strip.data() + ((size_t)(ib * nt + t) * n) * V;
                        std::memcpy(d, xs + ((size_t)iy * pw + ix) * V, sizeof(float) * V * n);
                    }
                }
                for (int ob = 0; ob < ocb; ++ob) {
                    const long wlen = (long)icb * V * nt * V;
                    Row rw{yb.data() + ((size_t)ob * oh + oy) * ow * V, q, 2, n,
                           strip.data(), (long)nt * n * V, (long)n * V, 1, icb, c, nt,
                           nt ? wph[a][b].data() + ob * wlen : nullptr, bp.data() + (size_t)ob * V};
                    if (nt) dispatch(V, rw);
                    else {
                        for (int j = 0; j < n; ++j)
                            std::memcpy(rw.out + (size_t)(q + 2 * j) * V, rw.bias, sizeof(float) * V);
                    }
                }
            }
        }
    }
    from_blocked(yb.data(), out_ch, oh, ow, V, y);
    return 0;
}

}  // extern "C"
