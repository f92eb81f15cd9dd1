// CPU oracle for the JPEG AI synthesis hot path. TEST INFRASTRUCTURE ONLY.
//
// This file restates, in plain C++ loops, the numeric contract of the reference's
// `nn::reference` layers and the elementwise / attention math of `nn::fast::math`. It exists so
// that the tests, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` have a
// checker. Nothing in the product library links, loads or calls it.
//
// Contract being restated (reference `src/nn/mod.rs:3-29`):
//   * convolution: acc = bias; for ic { for ky { for kx { acc = fma(w, x, acc) } } } over a
//     zero-padded input, padding taps included;
//   * transposed convolution: the same over the taps whose stride parity reaches the output,
//     ky and kx ascending;
//   * everything else: elementwise IEEE arithmetic, op by op, never contracted.
// Built with -ffp-contract=off so that only the explicit std::fma calls fuse.
//
// Tensors are planar [c][h][w] float32 (the reference's `Tensor<f32>`, `src/tensor.rs:12`).

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

extern "C" {

// ---------------------------------------------------------------------------------------------
// Convolution. Follows `reference::zero_pad`/`conv_plane`/`conv2d` (src/nn/reference.rs:17-133).
// `extra` = [top, left, bottom, right] zero padding on top of the layer's own, as
// `ConvLayer::with_extra_pad` (src/nn/fast/layers.rs:36, fallback path :104-118).
// Returns 0, or -1 for an inconsistent geometry (the reference's InvalidArgument / Model errors).
// ---------------------------------------------------------------------------------------------
int or_conv2d(const float* x, int c, int h, int w, const float* weight, const float* bias,
              int out_ch, int kh, int kw, int stride, int pad_h, int pad_w, int groups,
              const int* extra, float* y) {
    const int et = extra ? extra[0] : 0, el = extra ? extra[1] : 0;
    const int eb = extra ? extra[2] : 0, er = extra ? extra[3] : 0;
    if (groups <= 0 || c % groups || out_ch % groups || stride <= 0 || kh <= 0 || kw <= 0)
        return -1;
    const int ih = h + et + eb, iw = w + el + er;
    const int ph = ih + 2 * pad_h, pw = iw + 2 * pad_w;
    if (ph < kh || pw < kw) return -1;
    const int oh = (ph - kh) / stride + 1, ow = (pw - kw) / stride + 1;
    // zero_pad (reference.rs:17-27) of the extra-padded input.
    std::vector<float> xp((size_t)c * ph * pw, 0.0f);
    for (int ch = 0; ch < c; ++ch)
        for (int yy = 0; yy < h; ++yy)
            std::memcpy(&xp[((size_t)ch * ph + yy + et + pad_h) * pw + el + pad_w],
                        &x[((size_t)ch * h + yy) * w], sizeof(float) * w);
    const int icg = c / groups, ocg = out_ch / groups;
    const int wlen = icg * kh * kw;
#pragma omp parallel for schedule(dynamic, 1)
    for (int oc = 0; oc < out_ch; ++oc) {
        const int ic0 = (oc / ocg) * icg;
        const float* wt = weight + (size_t)oc * wlen;
        const float b = bias ? bias[oc] : 0.0f;
        std::vector<float> acc(ow);
        for (int oy = 0; oy < oh; ++oy) {
            for (int ox = 0; ox < ow; ++ox) acc[ox] = b;
            for (int i = 0; i < icg; ++i) {
                const float* plane = &xp[(size_t)(ic0 + i) * ph * pw];
                for (int ky = 0; ky < kh; ++ky) {
                    const float* row = plane + (size_t)(oy * stride + ky) * pw;
                    for (int kx = 0; kx < kw; ++kx) {
                        const float wv = wt[(i * kh + ky) * kw + kx];
                        if (stride == 1) {
                            const float* r = row + kx;
                            for (int ox = 0; ox < ow; ++ox) acc[ox] = std::fma(wv, r[ox], acc[ox]);
                        } else {
                            for (int ox = 0; ox < ow; ++ox)
                                acc[ox] = std::fma(wv, row[ox * stride + kx], acc[ox]);
                        }
                    }
                }
            }
            std::memcpy(&y[((size_t)oc * oh + oy) * ow], acc.data(), sizeof(float) * ow);
        }
    }
    return 0;
}

// Output size helper for callers (reference `Conv2d::out_size`, src/nn/mod.rs:124-129).
void or_conv2d_out_size(int h, int w, int kh, int kw, int stride, int pad_h, int pad_w,
                        const int* extra, int* oh, int* ow) {
    const int ih = h + (extra ? extra[0] + extra[2] : 0), iw = w + (extra ? extra[1] + extra[3] : 0);
    *oh = (ih + 2 * pad_h - kh) / stride + 1;
    *ow = (iw + 2 * pad_w - kw) / stride + 1;
}

// ---------------------------------------------------------------------------------------------
// Transposed convolution. Follows `reference::conv_transpose_plane`/`conv_transpose2d`
// (src/nn/reference.rs:155-236): input zero-padded by ext = ceil(k/s)+1 on every side; per
// output element, acc = bias; for ic { for ky { if parity reaches { for kx { ... fma } } } }.
// Weight layout [in][out][k][k] (src/nn/mod.rs:134-136); out = (n-1)*s + k + out_pad - 2*pad.
// ---------------------------------------------------------------------------------------------
int or_conv_transpose2d(const float* x, int c, int h, int w, const float* weight,
                        const float* bias, int out_ch, int k, int stride, int pad, int out_pad,
                        float* y) {
    if (stride <= 0 || k <= 0 || pad >= k || out_pad >= stride || h <= 0 || w <= 0) return -1;
    const int oh = (h - 1) * stride + k + out_pad - 2 * pad;
    const int ow = (w - 1) * stride + k + out_pad - 2 * pad;
    const int ext = (k + stride - 1) / stride + 1;
    const int ph = h + 2 * ext, pw = w + 2 * ext;
    std::vector<float> xp((size_t)c * ph * pw, 0.0f);
    for (int ch = 0; ch < c; ++ch)
        for (int yy = 0; yy < h; ++yy)
            std::memcpy(&xp[((size_t)ch * ph + yy + ext) * pw + ext], &x[((size_t)ch * h + yy) * w],
                        sizeof(float) * w);
#pragma omp parallel for schedule(dynamic, 1)
    for (int oc = 0; oc < out_ch; ++oc) {
        const float b = bias ? bias[oc] : 0.0f;
        for (int oy = 0; oy < oh; ++oy)
            for (int ox = 0; ox < ow; ++ox) {
                float acc = b;
                for (int ic = 0; ic < c; ++ic) {
                    const float* plane = &xp[(size_t)ic * ph * pw];
                    const float* wb = weight + ((size_t)ic * out_ch + oc) * k * k;
                    for (int ky = 0; ky < k; ++ky) {
                        const int ty = oy + pad + ext * stride - ky;
                        if (ty % stride) continue;
                        const float* row = plane + (size_t)(ty / stride) * pw;
                        for (int kx = 0; kx < k; ++kx) {
                            const int tx = ox + pad + ext * stride - kx;
                            if (tx % stride) continue;
                            acc = std::fma(wb[ky * k + kx], row[tx / stride], acc);
                        }
                    }
                }
                y[((size_t)oc * oh + oy) * ow + ox] = acc;
            }
    }
    return 0;
}

// `reference::pixel_shuffle` (src/nn/reference.rs:353-376): out channel oc at
// (y*r+dy, x*r+dx) is input channel oc*r*r + dy*r + dx at (y, x).
int or_pixel_shuffle(const float* x, int c, int h, int w, int r, float* y) {
    if (r <= 0 || c % (r * r)) return -1;
    const int oc_n = c / (r * r);
#pragma omp parallel for schedule(static)
    for (int oc = 0; oc < oc_n; ++oc)
        for (int dy = 0; dy < r; ++dy)
            for (int dx = 0; dx < r; ++dx) {
                const float* src = x + (size_t)(oc * r * r + dy * r + dx) * h * w;
                for (int yy = 0; yy < h; ++yy)
                    for (int xx = 0; xx < w; ++xx)
                        y[((size_t)oc * h * r + yy * r + dy) * w * r + xx * r + dx] = src[yy * w + xx];
            }
    return 0;
}

// ---------------------------------------------------------------------------------------------
// Elementwise operations (src/nn/reference.rs:339-350, src/nn/fast/layers.rs:174-229,
// src/model/hyper_encoder.rs:21-30, src/model/synthesis.rs:187-192). Each element is computed
// on its own, so the OpenMP split over elements changes no result.
// ---------------------------------------------------------------------------------------------
// f32::max(x, 0): a NaN input gives 0.
void or_relu(float* x, long n) {
#pragma omp parallel for simd schedule(static)
    for (long i = 0; i < n; ++i) x[i] = std::fmax(x[i], 0.0f);
}
// f32::clamp(0, 6): NaN stays NaN.
void or_relu6(float* x, long n) {
#pragma omp parallel for schedule(static)
    for (long i = 0; i < n; ++i) {
        float v = x[i];
        if (v < 0.0f) v = 0.0f;
        if (v > 6.0f) v = 6.0f;
        x[i] = v;
    }
}
void or_add(float* dst, const float* src, long n) {
#pragma omp parallel for simd schedule(static)
    for (long i = 0; i < n; ++i) dst[i] += src[i];
}
// `x *= 1 + mask`: an add then a multiply, never fused (layers.rs:195-201).
void or_gate(float* x, const float* mask, long n) {
#pragma omp parallel for simd schedule(static)
    for (long i = 0; i < n; ++i) { const float g = 1.0f + mask[i]; x[i] = x[i] * g; }
}
// `if v < 0 { v *= 0.01 }` (hyper_encoder.rs:24-30).
void or_leaky_relu(float* x, long n) {
#pragma omp parallel for schedule(static)
    for (long i = 0; i < n; ++i) if (x[i] < 0.0f) x[i] = x[i] * 0.01f;
}
void or_mul(float* a, const float* b, long n) {
#pragma omp parallel for simd schedule(static)
    for (long i = 0; i < n; ++i) a[i] = a[i] * b[i];
}
// `(x * 128 + 127.5).clamp(0, 255)` (synthesis.rs:187-192).
void or_denormalize(float* x, long n) {
#pragma omp parallel for schedule(static)
    for (long i = 0; i < n; ++i) {
        float v = x[i] * 128.0f;
        v = v + 127.5f;
        if (v < 0.0f) v = 0.0f;
        if (v > 255.0f) v = 255.0f;
        x[i] = v;
    }
}

// ---------------------------------------------------------------------------------------------
// Cephes expf as straight IEEE operations (src/nn/fast/math.rs:28-62).
// ---------------------------------------------------------------------------------------------
static const float kLog2e = 1.44269504088896340736f;
static const float kLn2Hi = 0.693359375f;
static const float kLn2Lo = -2.12194440e-4f;
static const float kP[6] = {1.9875691500e-4f, 1.3981999507e-3f, 8.3334519073e-3f,
                            4.1665795894e-2f, 1.6666665459e-1f, 5.0000001201e-1f};

float or_exp(float x) {
    if (x < -87.0f) x = -87.0f;
    if (x > 88.0f) x = 88.0f;
    float t = x * kLog2e;
    t = t + 0.5f;
    const float n = std::floor(t);
    float r = x - n * kLn2Hi;
    r = r - n * kLn2Lo;
    float p = kP[0];
    for (int i = 1; i < 6; ++i) { p = p * r; p = p + kP[i]; }
    float y = p * (r * r);
    y = y + r;
    y = y + 1.0f;
    const int ni = std::isnan(n) ? 0 : (int)n;  // Rust `as i32` maps NaN to 0
    uint32_t bits = (uint32_t)(ni + 127) << 23;
    float scale;
    std::memcpy(&scale, &bits, 4);
    return y * scale;
}

void or_exp_slice(float* x, long n) {
#pragma omp parallel for schedule(static)
    for (long i = 0; i < n; ++i) x[i] = or_exp(x[i]);
}
// `1 / (1 + exp(-x))` (math.rs:67-71).
void or_sigmoid(float* x, long n) {
#pragma omp parallel for schedule(static)
    for (long i = 0; i < n; ++i) { const float e = or_exp(-x[i]); x[i] = 1.0f / (1.0f + e); }
}
// `a = (a > 0 ? a : exp(a) - 1) * b` (math.rs:74-80).
void or_elu_gate(float* a, const float* b, long n) {
#pragma omp parallel for schedule(static)
    for (long i = 0; i < n; ++i) {
        const float e = or_exp(a[i]) - 1.0f;
        const float elu = a[i] > 0.0f ? a[i] : e;
        a[i] = elu * b[i];
    }
}

// ---------------------------------------------------------------------------------------------
// Layer norm over channels per position, f64 sums (math.rs:423-448).
// ---------------------------------------------------------------------------------------------
int or_layer_norm_channels(float* x, int c, int h, int w, const float* weight, const float* bias) {
    if (c <= 0) return -1;
    const long n = (long)h * w;
    // Positions are independent (each one's channel sums run in channel order): OpenMP splits
    // the map into blocks of positions.
    constexpr long B = 256;
#pragma omp parallel for schedule(static)
    for (long b0 = 0; b0 < n; b0 += B) {
        const long nb = std::min(B, n - b0);
        double mean[B], var[B];
        float m32[B], den[B];
        for (long i = 0; i < nb; ++i) mean[i] = var[i] = 0.0;
        for (int ch = 0; ch < c; ++ch) {
            const float* p = x + (size_t)ch * n + b0;
            for (long i = 0; i < nb; ++i) mean[i] += (double)p[i];
        }
        for (long i = 0; i < nb; ++i) mean[i] /= (double)c;
        for (int ch = 0; ch < c; ++ch) {
            const float* p = x + (size_t)ch * n + b0;
            for (long i = 0; i < nb; ++i) { const double d = (double)p[i] - mean[i]; var[i] += d * d; }
        }
        for (long i = 0; i < nb; ++i) {
            m32[i] = (float)mean[i];
            den[i] = std::sqrt((float)(var[i] / (double)c) + 1e-5f);
        }
        for (int ch = 0; ch < c; ++ch) {
            float* p = x + (size_t)ch * n + b0;
            for (long i = 0; i < nb; ++i) {
                float v = p[i] - m32[i];
                v = v / den[i];
                v = v * weight[ch];
                p[i] = v + bias[ch];
            }
        }
    }
    return 0;
}

// f64 dot product with eight interleaved accumulators combined pairwise (math.rs:452-465).
double or_dot8(const float* a, const float* b, long n) {
    double acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const long full = n / 8 * 8;
    for (long i = 0; i < full; i += 8)
        for (int l = 0; l < 8; ++l) acc[l] += (double)a[i + l] * (double)b[i + l];
    for (long i = full; i < n; ++i) acc[i - full] += (double)a[i] * (double)b[i];
    return ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
}

// Channel attention (`tam.py::Attention` without its projection; math.rs:512-603, exact
// precision). qkv [3*dim][h][w] planar; out [dim][h][w]; attn_out (optional) [dim][c].
int or_channel_attention(const float* qkv, int c3, int h, int w, int heads, const float* temperature,
                         float* out, float* attn_out) {
    if (heads <= 0 || c3 % (3 * heads)) return -1;
    const int dim = c3 / 3, c = dim / heads;
    const long n = (long)h * w;
    std::vector<float> qk(qkv, qkv + (size_t)2 * dim * n);
#pragma omp parallel for
    for (int row = 0; row < 2 * dim; ++row) {
        float* r = &qk[(size_t)row * n];
        const float norm = (float)std::sqrt(or_dot8(r, r, n));
        const float d = norm > 1e-12f ? norm : 1e-12f;
        for (long i = 0; i < n; ++i) r[i] = r[i] / d;
    }
    const float* q = qk.data();
    const float* k = qk.data() + (size_t)dim * n;
    const float* v = qkv + (size_t)2 * dim * n;
    std::vector<float> attn((size_t)dim * c);
#pragma omp parallel for
    for (int ri = 0; ri < dim; ++ri) {
        const int head = ri / c;
        float* row = &attn[(size_t)ri * c];
        float mx = -INFINITY;
        for (int j = 0; j < c; ++j) {
            row[j] = (float)or_dot8(q + (size_t)ri * n, k + (size_t)(head * c + j) * n, n) * temperature[head];
            mx = std::fmax(mx, row[j]);
        }
        for (int j = 0; j < c; ++j) row[j] = or_exp(row[j] - mx);
        double sum = 0.0;
        for (int j = 0; j < c; ++j) sum += (double)row[j];
        const float s = (float)sum;
        for (int j = 0; j < c; ++j) row[j] = row[j] / s;
    }
#pragma omp parallel for
    for (int ri = 0; ri < dim; ++ri) {
        const int head = ri / c;
        std::vector<double> acc(n, 0.0);
        for (int j = 0; j < c; ++j) {
            const double a = (double)attn[(size_t)ri * c + j];
            const float* vv = v + (size_t)(head * c + j) * n;
            for (long i = 0; i < n; ++i) acc[i] += a * (double)vv[i];
        }
        for (long i = 0; i < n; ++i) out[(size_t)ri * n + i] = (float)acc[i];
    }
    if (attn_out) std::memcpy(attn_out, attn.data(), sizeof(float) * attn.size());
    return 0;
}

// ---------------------------------------------------------------------------------------------
// Output quantisation: rintf(convert_range(clamp(x,0,255), 255, max)).clamp(0, max)
// (src/decoder/output.rs:38-40, :325-342). rint in the default round-half-even mode.
// ---------------------------------------------------------------------------------------------
void or_quantize_plane(const float* x, long n, int bit_depth, uint16_t* out) {
    const float mx = (float)((1u << bit_depth) - 1);
    for (long i = 0; i < n; ++i) {
        float v = x[i];
        if (v < 0.0f) v = 0.0f;
        if (v > 255.0f) v = 255.0f;
        v = v / 255.0f;
        v = v * mx;
        v = std::rint(v);
        if (v < 0.0f) v = 0.0f;
        if (v > mx) v = mx;
        out[i] = (uint16_t)v;
    }
}

// ---------------------------------------------------------------------------------------------
// f16 weight rounding (src/weights/f16.rs:12-67): pure-integer RNE f32 -> f16 and exact upcast.
// ---------------------------------------------------------------------------------------------
uint16_t or_f32_to_f16(float v) {
    uint32_t b;
    std::memcpy(&b, &v, 4);
    const uint16_t sign = (uint16_t)((b >> 16) & 0x8000);
    const int exp = (int)((b >> 23) & 0xff);
    const uint32_t mant = b & 0x007fffff;
    if (exp == 255) {
        uint16_t payload = (uint16_t)((mant >> 13) | 0x200);
        if (payload < 1) payload = 1;
        return (uint16_t)(sign | 0x7c00 | (mant ? payload : 0));
    }
    const int e = exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00);
    if (e <= 0) {
        if (e < -10) return sign;
        const uint32_t m = mant | 0x00800000;
        const uint32_t shift = (uint32_t)(14 - e);
        const uint32_t dropped = m & ((1u << shift) - 1);
        const uint32_t half = 1u << (shift - 1);
        uint32_t r = m >> shift;
        if (dropped > half || (dropped == half && (r & 1))) r += 1;
        return (uint16_t)(sign | r);
    }
    const uint32_t dropped = mant & 0x1fff;
    uint32_t r = mant >> 13;
    if (dropped > 0x1000 || (dropped == 0x1000 && (r & 1))) r += 1;
    return (uint16_t)(sign | (((uint32_t)e << 10) + r));
}

float or_f16_to_f32(uint16_t hbits) {
    const uint32_t sign = ((uint32_t)hbits & 0x8000) << 16;
    const uint32_t exp = (hbits >> 10) & 0x1f;
    const uint32_t mant = hbits & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        float sub = (float)mant * 5.9604644775390625e-08f;  // 2^-24, exact
        std::memcpy(&bits, &sub, 4);
        bits |= sign;
    } else if (exp == 31) {
        bits = sign | 0x7f800000 | (mant << 13);
    } else {
        bits = sign | ((exp + 112) << 23) | (mant << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

void or_f16_round_trip(const float* x, long n, float* y) {
    for (long i = 0; i < n; ++i) y[i] = or_f16_to_f32(or_f32_to_f16(x[i]));
}

// ---------------------------------------------------------------------------------------------
// Output stage (src/decoder/output.rs). Chroma resampling restates PyTorch's CPU kernels as the
// reference pins them operation for operation:
//   * bicubic, align_corners (`resize_bicubic`, :100-147): per output coordinate scale =
//     (in - 1) / (out - 1), real = scale * dst, base = floor(real), t = real - base, taps
//     clamp(base - 1 + k); A = -0.75 cubic weights with the fused forms of :64-79; four
//     horizontal dot4 = fma(x3, c3, fma(x2, c2, fma(x0, c0, x1 * c1))) (:85-90), then the
//     vertical dot4 over them;
//   * bilinear, align_corners (`nn::resize_bilinear`, src/nn/resample.rs:22-69): i0 = (int)real,
//     i1 = i0 + (i0 < in - 1), l1 = real - i0, l0 = 1 - l1; equal sizes map straight through;
//     pre-multiplied corner weights accumulated fma(p0, a, p1 * b), fma(p2, c, _), fma(p3, d, _).
// Planes are [c][h][w]; returns 0, or -1 for an empty input.
// ---------------------------------------------------------------------------------------------
static float or_cubic1(float x) {
    const float A = -0.75f;
    const float p = std::fma(A + 2.0f, x, -(A + 3.0f));
    return std::fma(p * x, x, 1.0f);
}
static float or_cubic2(float x) {
    const float A = -0.75f;
    float p = std::fma(A, x, -5.0f * A);
    p = std::fma(p, x, 8.0f * A);
    return std::fma(p, x, -4.0f * A);
}
static float or_dot4(const float* x, const float* c) {
    float acc = x[1] * c[1];
    acc = std::fma(x[0], c[0], acc);
    acc = std::fma(x[2], c[2], acc);
    return std::fma(x[3], c[3], acc);
}
static void or_cubic_taps(int dst, int in_len, int out_len, int* idx, float* wt) {
    const float scale = out_len > 1 ? (float)(in_len - 1) / (float)(out_len - 1) : 0.0f;
    const float real = scale * (float)dst;
    const float basef = std::floor(real);
    const float t = real - basef;
    const int base = (int)basef;
    for (int k = 0; k < 4; ++k) {
        int i = base - 1 + k;
        i = i < 0 ? 0 : (i > in_len - 1 ? in_len - 1 : i);
        idx[k] = i;
    }
    const float u = 1.0f - t;
    wt[0] = or_cubic2(t + 1.0f);
    wt[1] = or_cubic1(t);
    wt[2] = or_cubic1(u);
    wt[3] = or_cubic2(u + 1.0f);
}

int or_resize_bicubic(const float* src, int c, int h, int w, int oh, int ow, float* dst) {
    if (h <= 0 || w <= 0) return -1;
    std::vector<int> xi((size_t)ow * 4), yi((size_t)oh * 4);
    std::vector<float> xw((size_t)ow * 4), yw((size_t)oh * 4);
    for (int x = 0; x < ow; ++x) or_cubic_taps(x, w, ow, &xi[(size_t)x * 4], &xw[(size_t)x * 4]);
    for (int y = 0; y < oh; ++y) or_cubic_taps(y, h, oh, &yi[(size_t)y * 4], &yw[(size_t)y * 4]);
    for (int ch = 0; ch < c; ++ch) {
        const float* sp = src + (size_t)ch * h * w;
        float* dp = dst + (size_t)ch * oh * ow;
        for (int y = 0; y < oh; ++y)
            for (int x = 0; x < ow; ++x) {
                float rows[4];
                for (int k = 0; k < 4; ++k) {
                    const float* row = sp + (size_t)yi[(size_t)y * 4 + k] * w;
                    const int* ix = &xi[(size_t)x * 4];
                    const float v[4] = {row[ix[0]], row[ix[1]], row[ix[2]], row[ix[3]]};
                    rows[k] = or_dot4(v, &xw[(size_t)x * 4]);
                }
                dp[(size_t)y * ow + x] = or_dot4(rows, &yw[(size_t)y * 4]);
            }
    }
    return 0;
}

static void or_linear_taps(int dst, int in_len, int out_len, int* i0, int* i1, float* l0, float* l1) {
    if (in_len == out_len) {
        *i0 = *i1 = dst;
        *l0 = 1.0f;
        *l1 = 0.0f;
        return;
    }
    const float scale = out_len > 1 ? (float)(in_len - 1) / (float)(out_len - 1) : 0.0f;
    const float real = scale * (float)dst;
    const int a = (int)real;
    *i0 = a;
    *i1 = a + (a < in_len - 1 ? 1 : 0);
    *l1 = real - (float)a;
    *l0 = 1.0f - *l1;
}

int or_resize_bilinear(const float* src, int c, int h, int w, int oh, int ow, float* dst) {
    if (h <= 0 || w <= 0 || oh <= 0 || ow <= 0) return -1;
    for (int ch = 0; ch < c; ++ch) {
        const float* sp = src + (size_t)ch * h * w;
        float* dp = dst + (size_t)ch * oh * ow;
        for (int y = 0; y < oh; ++y) {
            int y0, y1;
            float h0, h1;
            or_linear_taps(y, h, oh, &y0, &y1, &h0, &h1);
            for (int x = 0; x < ow; ++x) {
                int x0, x1;
                float w0, w1;
                or_linear_taps(x, w, ow, &x0, &x1, &w0, &w1);
                const float p0 = h0 * w0, p1 = h0 * w1, p2 = h1 * w0, p3 = h1 * w1;
                const float* r0 = sp + (size_t)y0 * w;
                const float* r1 = sp + (size_t)y1 * w;
                float acc = std::fma(p0, r0[x0], p1 * r0[x1]);
                acc = std::fma(p2, r1[x0], acc);
                dp[(size_t)y * ow + x] = std::fma(p3, r1[x1], acc);
            }
        }
    }
    return 0;
}

// `to_rgb_planes_owned_par` (src/decoder/output.rs:232-257) on 4:4:4 planes: BT.709 constants
// combined in f64 and narrowed to f32 (:27-33, :225-228); convert_range(x, a, b) =
// ((x - 0) / a) * b + 0 (:36-40); clamp to [0, 255]. In place is allowed.
static float or_convert_range(float x, float in_max, float out_max) {
    float v = x - 0.0f;
    v = v / in_max;
    v = v * out_max;
    return v + 0.0f;
}
static float or_clamp255(float v) { return v < 0.0f ? 0.0f : (v > 255.0f ? 255.0f : v); }

void or_yuv_to_rgb(const float* y, const float* u, const float* v, long n, float* r, float* g,
                   float* b) {
    const double KR = 0.2126, KG = 0.7152, KB = 0.0722, KBY = 1.8556, KRY = 1.5748;
    const float kry = (float)KRY, kby = (float)KBY;
    const float gu = (float)(KB * KBY / KG), gv = (float)(KR * KRY / KG);
    for (long i = 0; i < n; ++i) {
        const float yy = or_convert_range(y[i], 255.0f, 1.0f);
        const float uu = or_convert_range(u[i], 255.0f, 1.0f) - 0.5f;
        const float vv = or_convert_range(v[i], 255.0f, 1.0f) - 0.5f;
        const float rv = yy + kry * vv;
        float gvv = yy - gu * uu;
        gvv = gvv - gv * vv;
        const float bv = yy + kby * uu;
        r[i] = or_clamp255(or_convert_range(rv, 1.0f, 255.0f));
        g[i] = or_clamp255(or_convert_range(gvv, 1.0f, 255.0f));
        b[i] = or_clamp255(or_convert_range(bv, 1.0f, 255.0f));
    }
}

// `quantize_par` (src/decoder/output.rs:407-437): interleaved [n][3] samples,
// convert_range(x, 255, max), round half to even, clamp to [0, max].
void or_quantize_rgb(const float* r, const float* g, const float* b, long n, int bit_depth,
                     uint16_t* out) {
    const float mx = (float)((1u << bit_depth) - 1);
    const float* pl[3] = {r, g, b};
    for (long i = 0; i < n; ++i)
        for (int k = 0; k < 3; ++k) {
            float v = std::rint(or_convert_range(pl[k][i], 255.0f, mx));
            v = v < 0.0f ? 0.0f : (v > mx ? mx : v);
            out[i * 3 + k] = (uint16_t)v;
        }
}

}  // extern "C"
