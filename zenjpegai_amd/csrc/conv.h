// Launch description of the implicit-GEMM convolution kernels (host and device).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "device.h"

namespace zjai {

// Activation applied to the accumulator before the residual operation.
enum Act : int { ACT_NONE = 0, ACT_RELU = 1, ACT_LEAKY = 2, ACT_SIGMOID = 3 };

// Residual operation of the epilogue (r1, r2 are views with the output's geometry):
//   RES_ADD  y = a + r1                   (ResidualBlock / LightResidualBlock / TAM skip)
//   RES_GATE y = r1 * (1 + a)             (ResAU gate, src/nn/fast/layers.rs:195-201)
//   RES_CAB  y = r1 * sigmoid(a) + r2     (CAB, src/model/attention.rs:130-137)
//   RES_MUL  y = r1 * a
enum Res : int { RES_NONE = 0, RES_ADD = 1, RES_GATE = 2, RES_CAB = 3, RES_MUL = 4 };

// Where the epilogue writes.
enum Out : int { OUT_NHWC = 0, OUT_PLANE = 1 };

struct ConvParams {
    // Input view and its valid extent (reads outside [0,H) x [0,W) are zero padding).
    View x;
    int H, W;
    int N;  // batch items (tiles)
    // Output extent in conv-output coordinates (before pixel shuffle).
    int OH, OW;
    View y;  // OUT_NHWC destination (after pixel shuffle)
    // Packed weights: [phase][group][chunk][nblk][tap][16][CK] in the storage type; bias f32.
    // w_bstride > 0: one packed weight per batch item (the folded attention projection).
    const void* w;
    long long w_bstride;
    const float* bias;
    int cin_g, cout_g, groups, nchunks, nblk_g, ntiles;
    int gx, gy;  // spatial tile grid (set by the launcher)
    long long phase_stride;  // elements between phases (transposed conv)
    int pad_t, pad_l;
    int relu6_in;  // clamp(x, 0, 6) on load (ResAU's relu6)
    // Epilogue.
    int act, res;
    View r1, r2;
    int ps;  // pixel shuffle factor (1 = none)
    int out_mode;
    // OUT_PLANE: planar destination. Channel c of the (shuffled) output of batch item b goes to
    // plane + c * pl_cstride; the kept window [win_y0[b], +win_h[b]) x [win_x0[b], +win_w[b]) of
    // the output lands at (dst_y0[b], dst_x0[b]), keeping rows/cols that are multiples of sv / sh.
    void* plane;
    long long pl_row, pl_cstride;
    int sv, sh;
    int denorm;     // x * 128 + 127.5 clamped to [0, 255]
    int bit_depth;  // 0: store f32; else quantise to u16 at this depth
    int win_y0[MAXB], win_x0[MAXB], win_h[MAXB], win_w[MAXB], dst_y0[MAXB], dst_x0[MAXB];
    // Transposed conv (stride 2): tap tables per output phase (py * 2 + px).
    int ntaps[4];
    int tap_dy[4][4], tap_dx[4][4];
};

// Kernel configuration: waves along channels (WC) x along rows (WP), each wave CF channel
// blocks of 16 x PF output rows of 16 columns.
struct TileCfg {
    int wc, wp, cf, pf;
};

enum ConvKind : int { CK_1x1 = 0, CK_2x2 = 1, CK_3x3 = 2, CK_3x3_S2 = 3, CK_T3 = 4 };

hipError_t launch_conv(int kind, int dtype, TileCfg cfg, const ConvParams& p, hipStream_t s);

// Stride-2 transposed conv with 3x3 kernels (9 taps over the four output phases), all four
// phases of a tile in one workgroup: p.w is the phase-merged packing [chunk][nblk][9][16][CK]
// (taps phase by phase, each phase's taps in its table order), p.ntiles = nblk_g / 4; NHWC
// output without pixel shuffle, no relu6 on load.
hipError_t launch_conv_tr_merged(int dtype, const ConvParams& p, hipStream_t s);
// The per-phase tap counts conv_tr_merged is instantiated for (3x3 kernels, stride 2).
bool conv_tr_merged_taps_supported(const int (&ntaps)[4]);
constexpr int TR_MERGED_TAPS = 9;
constexpr int TR_MERGED_NB = 4;

// Dense stride-1 3x3 convolution in f16 / bf16 on 32x32x16 MFMAs (conv32.hip): mt (128 or 64)
// output channels x 256 positions per workgroup, tiles tw (32 or 16) columns wide; p.w is the
// packing [cin / 16][cout / mt][9][2][mt][8] of the storage type, p.cin_g 64 or 128,
// groups 1, NHWC output without pixel shuffle, no relu6 on load.
hipError_t launch_conv3x3_m32(int dtype, int mt, int tw, const ConvParams& p, hipStream_t s);
int conv3x3_m32_width(int OH, int OW);

// 1x1 layers (stride 1, no padding, one group) as a GEMM over row-major positions with a
// ring of direct-LDS chunk loads (conv1x1.hip); p.w is the implicit-GEMM packing, p.cout_g a
// multiple of 64, 16-byte aligned input views, no relu6 on load. Results are bit-identical to
// launch_conv on the same layer. conv1x1_ring_ok: whether p qualifies.
hipError_t launch_conv1x1_ring(int dtype, const ConvParams& p, hipStream_t s);
bool conv1x1_ring_ok(const ConvParams& p, int dtype);
int conv1x1_ring_nb(const ConvParams& p);

// Stride-2 transposed conv with cout <= 8 on the vector ALUs (coutp = cout rounded up to 1, 2, 4
// or 8); wn is [cin][phase][tap][coutp] f32. Uses p's input view, output geometry, tap tables,
// bias and epilogue fields.
// convT_narrow_k3: whether launch_convT_narrow takes the 3x3 / padding-1 kernel for p.
bool convT_narrow_k3(int dtype, const ConvParams& p, int cin);
hipError_t launch_convT_narrow(int dtype, int coutp, const ConvParams& p, const float* wn, int cin,
                               hipStream_t s);
// The same layers in f16 / bf16 on 16x16x32 MFMAs when their taps are the 3x3 / padding-1 ones
// and cin is 64 or 128 (convT_mfma_k3); wm is [cin / 32][neighbour][row block][16][32] in the
// storage type (row = phase * coutp + output, zero where a phase does not read the neighbour).
bool convT_mfma_k3(int dtype, const ConvParams& p, int cin);
hipError_t launch_convT3_mfma(int dtype, int coutp, const ConvParams& p, const void* wm, int cin, hipStream_t s);

}  // namespace zjai
