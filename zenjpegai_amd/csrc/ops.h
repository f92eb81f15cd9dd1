// Bandwidth-bound kernels of the synthesis path (layout, elementwise, depthwise, layer norm,
// channel attention). Host-callable launchers; every one runs over N batch items (tiles).
#pragma once

#include <string>

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "device.h"

namespace zjai {

enum EltOp : int {
    EL_RELU = 0,     // max(x, 0)
    EL_RELU6 = 1,    // clamp(x, 0, 6)
    EL_LEAKY = 2,    // x < 0 ? 0.01 x : x
    EL_SIGMOID = 3,  // 1 / (1 + exp(-x))
    EL_ADD = 4,      // x = x + s
    EL_GATE = 5,     // x = x * (1 + s)
    EL_MUL = 6,      // x = x * s
    EL_ELU_GATE = 7, // x = elu(x) * s
};

// Per batch item origin of a latent window.
struct Windows {
    int x0[MAXB], y0[MAXB];
};

// Planar f32 [C][LH][LW] windows (x0[b], y0[b], w, h) -> NHWC view of dtype, N items.
hipError_t launch_planar_to_nhwc(const float* src, int C, int LH, int LW, const Windows& win, int N,
                                 int h, int w, View dst, int dtype, hipStream_t s);
// NHWC view -> planar f32 [N][C][h][w].
hipError_t launch_nhwc_to_planar(View src, int dtype, int N, int C, int h, int w, float* dst,
                                 hipStream_t s);
// x = op(x[, s]) over N x h x w x C.
hipError_t launch_eltwise(int op, View x, View src, int dtype, int N, int C, int h, int w,
                          hipStream_t s);
// NHWC copy of C channels over N x h x w (channel offsets / crops / concatenation).
hipError_t launch_copy(View src, View dst, int dtype, int N, int C, int h, int w, hipStream_t s);
// Pixel shuffle NHWC -> NHWC: out channel c at (y*r+dy, x*r+dx) = in channel c*r*r+dy*r+dx.
hipError_t launch_pixel_shuffle(View src, View dst, int dtype, int N, int C_out, int h, int w,
                                int r, hipStream_t s);
// Depthwise 3x3, stride 1, pad 1, weights [9][C] f32, optional bias. With elu_half > 0 the
// output keeps channels [0, elu_half) = elu(dw(c)) * dw(c + elu_half) (the FFN gate).
hipError_t launch_depthwise3x3(View src, View dst, int dtype, int N, int C, int h, int w,
                               const float* weight, const float* bias, int elu_half,
                               hipStream_t s);
// Layer norm over channels per position (f64 sums), src -> dst.
hipError_t launch_layer_norm(View src, View dst, int dtype, int N, int C, int h, int w,
                             const float* weight, const float* bias, hipStream_t s);
// The feed-forward half of a transformer block in one kernel (every storage type, dim 64 or
// 128): y = x + project_out(elu(dw(project_in(LN(x)))[:hid]) * dw(...)[hid:]), hid = 4 * dim.
// Weights: the packed 1x1 layers ([chunk][nblk][16][64 bytes], storage type) and the depthwise
// [9][2 * hid] f32. y must not alias x (neighbouring tiles read x over their halos).
struct FfnArgs {
    View x, y;
    int N, h, w;
    int gx, gy;  // tile grid (set by the launcher)
    const float* ln_w;
    const float* ln_b;
    const void* w_in;  // project_in: dim -> 2 * hid
    int nblk_in;
    const float* b_in;
    const float* dw_w;
    const float* dw_b;
    const void* w_out;  // project_out: hid -> dim
    int nblk_out;
    const float* b_out;
};
bool ffn_fused_supported(int dtype, int dim);
// ResAU (x * (1 + conv1x1(conv3x3_grouped(relu6(x))))) in one kernel for C = 32 or 64 channels in
// groups of 16, every storage type; w1 / w2 are the two layers' implicit-GEMM packings (one K
// chunk and one 16-row block per group for w1; nblk2 16-row blocks for w2). y must not alias x.
struct ResauArgs {
    View x, y;
    int N, h, w;
    int gx, gy;  // tile grid (set by the launcher)
    const void* w1;
    const void* w2;
    int nblk2;
};
bool resau_fused_supported(int C, int groups);
int resau_rows(int dtype, int N, int h, int w);
hipError_t launch_resau(int dtype, int C, const ResauArgs& p, hipStream_t s);
// The attention branch's qkv = depthwise3x3(conv1x1(LN(x))) (dim -> 3 dim) in one kernel
// (every storage type, dim 64 or 128); weights as FfnArgs. y must not alias x.
struct QkvArgs {
    View x, y;
    int N, h, w;
    int gx, gy;  // tile grid (set by the launcher)
    const float* ln_w;
    const float* ln_b;
    const void* w1;  // conv1: dim -> 3 dim, packed 1x1
    int nblk1;
    const float* b1;
    const float* dw_w;  // [9][3 dim]
    const float* dw_b;
};
bool qkv_fused_supported(int dtype, int dim);
hipError_t launch_qkv_fused(const QkvArgs& a, int dtype, int dim, hipStream_t s);
// Output stage (src/decoder/output.rs): align_corners resampling of planar f32 [c][h][w] planes
// and the BT.709 picture -> interleaved uint16 RGB (+ optional float planes [3][H][W]).
enum ResizeMode : int { RESIZE_BICUBIC = 0, RESIZE_BILINEAR = 1 };
hipError_t launch_resize(int mode, const float* src, int c, int h, int w, float* dst, int oh, int ow,
                         hipStream_t s);
hipError_t launch_picture_rgb(const float* y, int H, int W, const float* u, const float* v, int ch,
                              int cw, int bit_depth, uint16_t* rgb, float* rgbf, hipStream_t s);
hipError_t launch_ffn_fused(const FfnArgs& a, int dtype, int dim, hipStream_t s);
// Channel attention (src/nn/fast/math.rs:512-603), three phases per batch item:
// 1. per-head Gram partial sums over chunks of positions (f32 MFMA): qkv view holds 3*dim
//    channels; partial[N][nchunk][heads][c*c + 2c] f32 (c = dim / heads <= 32);
// 2. reduction (f64), normalisation, temperature and softmax -> attn [N][dim][c] f32;
// 3. fold with the output projection proj [dim][dim] into a packed 1x1 conv weight per item
//    (wpk + b * w_bstride).
int attention_gram_chunks(int h, int w);
// Whether the Gram kernel's LDS stage (64 16-bit or 32 f32 positions of 2 dim channels) fits the
// 160 KB of a CU for this dim: callers check it before their first launch.
bool attention_gram_fits(int dtype, int dim);
// Profile name of the Gram kernel launch_attention_gram runs for these operands, as the kernel
// symbol reads (k_attention_gram<__bf16, true, 2>: the fixed-offset staging form, two 16-channel
// blocks per head).
std::string attention_gram_name(const View& qkv, int dtype, int dim, int heads, int w);
hipError_t launch_attention_gram(View qkv, int dtype, int N, int dim, int heads, int h, int w,
                                 float* partial, hipStream_t s);
hipError_t launch_attention_softmax(const float* partial, int N, int nchunk, int dim, int heads,
                                    const float* temperature, float* attn, hipStream_t s);
hipError_t launch_attention_fold(const float* proj, const float* attn, int N, int dim, int heads,
                                 int dtype, int nblk, void* wpk, long long w_bstride,
                                 hipStream_t s);
// Zero `bytes` (a multiple of 4, 4-byte aligned) at p with a kernel.
hipError_t launch_zero(void* p, size_t bytes, hipStream_t s);
// Adds the non-finite f16 samples of an N x [h][w][C] view to slots[0 .. nslots) (nslots
// workgroups, each adding to its own slot).
hipError_t launch_count_f16_nonfinite(View v, int N, int C, int h, int w, unsigned long long* slots,
                                      int nslots, hipStream_t s);

// Latent reconstruction (src/decoder/reconstruct.rs:81-234), N regions of one shape per launch:
// int8 planar z_hat windows (per item origin) -> NHWC view of the storage type;
hipError_t launch_i8_planar_to_nhwc(const int8_t* z, int C, int ZH, int ZW, const Windows& win, int N, int h, int w,
                                    View dst, int dtype, hipStream_t s);
// context-model stage (py, px): st (N x hh x hw x C, the means) += residual in place, y_hat
// planar [N][C][H][W] written at the stage's samples; item b's residual window starts at
// (rwin.x0[b], rwin.y0[b]) of planes with the given row / plane strides;
hipError_t launch_mcm_stage(View st, int dtype, int N, int C, int hh, int hw, const float* res, long long res_row,
                            long long res_plane, const Windows& rwin, int H, int W, int py, int px, float* y_hat,
                            hipStream_t s);
// no context model: y_hat [N][C][H][W] = up-shuffled psi (N x ph x pw x 4C) + residual;
hipError_t launch_upshuffle_psi(View psi, int dtype, int N, int C, int ph, int pw, const float* res, long long res_row,
                                long long res_plane, const Windows& rwin, int H, int W, float* y_hat, hipStream_t s);
// region merges: a clamped rectangle of an NHWC tile (SH x SW) or of a planar f32 tile into a
// planar f32 destination [C][DH][DW].
hipError_t launch_assign_from_nhwc(View src, int dtype, int C, int SH, int SW, int oy, int ox, int h, int w,
                                   float* dst, int DH, int DW, int dy0, int dx0, hipStream_t s);
hipError_t launch_assign_planar(const float* src, int C, int SH, int SW, int oy, int ox, int h, int w, float* dst,
                                int DH, int DW, int dy0, int dx0, hipStream_t s);

// Analysis transforms (src/model/analysis.rs): normalised planar picture planes -> NHWC with the
// first replicate padding (Cp >= C channels, zeros beyond C); replicate padding NHWC -> NHWC;
// per-channel clipping of channels [0, n) in place.
hipError_t launch_normalize_pad(const float* x, int C, int H, int W, int Cp, int OH, int OW, View dst, int dtype,
                                hipStream_t s);
hipError_t launch_replicate_pad(View src, int dtype, int N, int C, int H, int W, View dst, int OH, int OW,
                                hipStream_t s);
hipError_t launch_clip_channels(View x, int dtype, int N, int C, int H, int W, int n, const float* lo,
                                const float* hi, hipStream_t s);

}  // namespace zjai
