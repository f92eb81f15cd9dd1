// Host runtime of the HIP synthesis backend: context (one stream), device buffer pool,
// activation tensors, packed layers, synthesis nets and pictures.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "conv.h"
#include "error.h"
#include "ops.h"
#include "../../include/zjai_hip.h"

namespace zjai {

#define ZJAI_HIP(call)                                                                        \
    do {                                                                                      \
        hipError_t e_ = (call);                                                               \
        if (e_ != hipSuccess)                                                                 \
            throw ::zjai::Error(e_ == hipErrorOutOfMemory ? ZJAI_E_LIMIT : ZJAI_E_DEVICE,     \
                                std::string(#call ": ") + hipGetErrorString(e_));             \
    } while (0)

inline int dtype_size(int dt) { return dt == DT_F32 ? 4 : 2; }
inline int round_up(int a, int b) { return (a + b - 1) / b * b; }
inline int ceil_div(int a, int b) { return (a + b - 1) / b; }

// Host-side failure injection (zjai_inject_failure): after `left` more events of the armed kind
// (FAULT_ALLOC: a pool allocation, cached or not; FAULT_LAUNCH: a kernel launch) the next one
// throws, once, the error a failed hipMalloc (LimitExceeded) or a failed launch (device) throws.
// Nothing reaches the device: the throw happens before the allocation or the launch.
enum FaultKind : int { FAULT_NONE = 0, FAULT_ALLOC = 1, FAULT_LAUNCH = 2 };
struct FaultPlan {
    int what = FAULT_NONE;
    long long left = 0;
    // Called once per event of `kind`: true when this event is the one to fail (then disarms).
    bool take(int kind) {
        if (what != kind) return false;
        if (left > 0) {
            --left;
            return false;
        }
        what = FAULT_NONE;
        return true;
    }
};

// Caching device allocator: freed blocks go back to a per-size free list and are reused, so a
// steady-state decode allocates nothing (the reference's buffer pool, src/nn/fast/tensor.rs:21-119,
// keeps its host buffers the same way).
class Pool {
public:
    void* alloc(size_t bytes);
    void release(void* p);
    void trim();
    // Hands every cached (free) block to the caller, who frees it with hipFree: a captured HIP
    // graph keeps the blocks its launches address out of later allocations.
    void surrender(std::vector<void*>& out);
    size_t in_use() const { return in_use_; }
    size_t peak() const { return peak_; }
    size_t cached() const { return cached_; }
    // Starts a new high-water mark at the bytes now in use.
    void reset_peak() { peak_ = in_use_; }
    std::shared_ptr<FaultPlan> faults;  // the root context's plan (shared with its lanes)
    ~Pool();

private:
    static size_t bucket(size_t bytes);
    std::multimap<size_t, void*> free_;
    std::map<void*, size_t> live_;
    size_t in_use_ = 0, peak_ = 0, cached_ = 0;
};

struct Context;

// Device activation: n batch items (tiles of one shape) of [h][w][c], NHWC. The pool block
// returns to the pool when the last tensor or view of it dies.
struct Tensor {
    Context* ctx = nullptr;
    void* base = nullptr;
    View v{};
    int dtype = DT_F32, n = 1, c = 0, h = 0, w = 0;
    std::shared_ptr<void> keep;  // keeps the underlying block alive for views
    int cs() const { return v.cs; }
};
using TensorP = std::shared_ptr<Tensor>;

// One profiled launch: kernel name, algorithmic FLOPs and HBM bytes, HIP events around it.
struct ProfRec {
    std::string name;
    double flops = 0.0, bytes = 0.0;
    hipEvent_t a = nullptr, b = nullptr;
};

struct Context {
    int device = 0;
    uint32_t flags = 0;  // ZJAI_CTX_* (read from the root context)
    hipStream_t stream = nullptr;
    // The pool is shared with every tensor allocated from it, so a tensor that outlives its
    // context (a caller destroying the context first) still returns its block to a live pool.
    std::shared_ptr<Pool> pool_owner = std::make_shared<Pool>();
    Pool& pool = *pool_owner;
    std::shared_ptr<FaultPlan> faults = std::make_shared<FaultPlan>();
    // ZJAI_CTX_COUNT_F16_RANGE: per-workgroup counts of non-finite f16 samples written, one
    // array per lane (each lane's scans run in its own stream order), summed by zjai_get_stats.
    unsigned long long* range_slots = nullptr;
    std::string last_error;
    volatile int stop = 0;
    uint64_t mem_limit = 0;  // zjai_ctx_set_memory_limit: device bytes a picture may need (0: none)
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    float last_ms = 0.0f;
    long long launches = 0;
    // Per-launch profiling (zjai_profile_begin / zjai_profile_end).
    bool profiling = false;
    std::vector<ProfRec> prof;
    std::vector<hipEvent_t> ev_pool;
    size_t ev_used = 0;

    // Lanes: sub-contexts on the same device, each with its own stream and buffer pool (a pool
    // block is only reused in the stream order of the lane that freed it). Independent work --
    // the tile batches of a picture -- runs on several lanes at once so that one batch's kernels
    // fill the tail of another's. Launch counts, profiling and the stop flag stay with the root.
    Context* root = nullptr;
    bool owns_stream = false;
    std::vector<std::unique_ptr<Context>> lanes;
    Context& lane(int i);
    Context& top() { return root ? *root : *this; }

    Context() { pool.faults = faults; }
    TensorP alloc(int n, int c, int h, int w, int dtype);
    void check_stop();
    hipEvent_t take_event();
    ~Context();
};

// Brackets one kernel launch: counts it and, while profiling, records events around it.
class LaunchScope {
public:
    LaunchScope(Context& c, const std::string& name, double flops, double bytes);
    ~LaunchScope();
    LaunchScope(const LaunchScope&) = delete;
    LaunchScope& operator=(const LaunchScope&) = delete;

private:
    Context& c_;
    long idx_ = -1;
};

// ZJAI_CTX_COUNT_F16_RANGE: adds the non-finite samples of an f16 tensor just written on ctx's
// stream to ctx's counters (no-op for other precisions or without the flag).
void count_f16_range(Context& ctx, const Tensor& t);
// Allocates and clears ctx's counters when the flag is set (count_f16_range does it on first use;
// a HIP graph capture does it beforehand, so that the clearing is not part of the graph).
void range_slots_init(Context& ctx);
constexpr int RANGE_SLOTS = 256;
// Sum of every lane's counters (synchronises the context's streams).
unsigned long long f16_range_total(Context& root);

// View of the top-left h x w corner (`BTensor::crop_par`, src/nn/fast/tensor.rs:349-367).
TensorP crop_view(const TensorP& t, int h, int w);
// View of channels [c0, c0 + n) of t.
TensorP channel_view(const TensorP& t, int c0, int n);

// A convolution packed for the implicit-GEMM kernels (PackedConv / PackedConvTranspose /
// PackedDepthwise equivalents).
struct Layer {
    bool transposed = false, depthwise = false;
    int cin = 0, cout = 0, kh = 0, kw = 0, stride = 1, pad_h = 0, pad_w = 0, groups = 1;
    int k = 0, pad = 0, out_pad = 0;
    int extra[4] = {0, 0, 0, 0};
    int dtype = DT_F32;
    int kind = 0;
    TileCfg cfg{};
    int nblk_g = 0, nchunks = 0;
    long long phase_stride = 0;
    int ntaps[4] = {0, 0, 0, 0}, tap_dy[4][4] = {}, tap_dx[4][4] = {};
    void* wpk = nullptr;       // packed weights (storage dtype)
    float* bias = nullptr;     // f32 [cout] or null
    float* dw_w = nullptr;     // depthwise [9][C]
    float* w_f32 = nullptr;    // f32 [cout][cin] copy (1x1 only, for attention folding)
    float* wn = nullptr;       // narrow transposed conv: [cin][phase][tap][coutp] f32
    void* wpk_m = nullptr;     // 3x3 transposed conv, all phases per workgroup: [chunk][nblk][9][16][CK]
    size_t wpk_m_bytes = 0;
    void* wpk32 = nullptr;     // dense stride-1 3x3, 16-bit: [cin / 16][cout / mt32][9][mt32][16]
    int mt32 = 0;              // output channels per workgroup of conv3x3_m32 (0: not eligible)
    int coutp = 0;             // cout rounded up to 1, 2, 4 or 8 (narrow transposed conv)
    void* wm16 = nullptr;      // narrow 3x3 transposed conv, 16-bit MFMA: [cin / 32][4][row block][16][32]
    size_t wm16_bytes = 0;
    size_t wpk_bytes = 0;
    size_t dev_bytes = 0;      // device bytes of every array above
    ~Layer();

    void out_size(int h, int w, int* oh, int* ow) const;
};
using LayerP = std::shared_ptr<Layer>;

// Tile shape the implicit-GEMM kernels use for a layer with cout_g outputs per group.
TileCfg conv_tile_cfg(int cout_g, int kind, int dtype);

LayerP make_conv(Context& ctx, int cin, int cout, int kh, int kw, int stride, int pad_h,
                 int pad_w, int groups, const float* weight, const float* bias,
                 const int extra[4], int dtype, bool keep_f32);
LayerP make_conv_transpose(Context& ctx, int cin, int cout, int k, int stride, int pad,
                           int out_pad, const float* weight, const float* bias, int dtype);

// Fused epilogue description for one conv launch. `w_batch` (with `w_bstride` elements between
// items) replaces the layer's packed weight with one weight per batch item.
struct Epilogue {
    int act = ACT_NONE, res = RES_NONE, ps = 1, relu6_in = 0;
    const Tensor* r1 = nullptr;
    const Tensor* r2 = nullptr;
    const void* w_batch = nullptr;
    long long w_bstride = 0;
};

// Planar picture destination of a last layer; windows per batch item.
struct PlaneOut {
    void* plane = nullptr;
    long long row = 0, cstride = 0;
    int sv = 1, sh = 1, denorm = 1, bit_depth = 0;
    int win_y0[MAXB] = {}, win_x0[MAXB] = {}, win_h[MAXB] = {}, win_w[MAXB] = {};
    int dst_y0[MAXB] = {}, dst_x0[MAXB] = {};
};

// Runs a layer on x. With `dst` null a new tensor is allocated; with `plane` set the output
// goes to the planar destination instead.
TensorP conv_forward(Context& ctx, const Layer& L, const TensorP& x, const Epilogue& e,
                     const TensorP& dst = nullptr, const PlaneOut* plane = nullptr);

std::string conv_kernel_name(int kind, int dtype, TileCfg c);
// "<base><T>" as profilers print the templated kernels of ops.hip.
inline std::string kname(const char* base, int dtype) {
    static const char* ty[] = {"float", "_Float16", "__bf16"};
    return std::string(base) + "<" + ty[dtype] + ">";
}

// Channel attention of qkv (3*dim channels, `heads` heads, device temperature) folded with the
// projection layer `proj` (a dense 1x1 dim -> dim layer holding its f32 weight): returns, per
// batch item, proj . blockdiag(attn) packed like proj's weight (`*w_bstride` elements apart), so
// proj run with these weights on the v channels of qkv yields
// project_out(channel_attention(qkv)).
std::shared_ptr<void> attention_fold(Context& ctx, const TensorP& qkv, int heads,
                                     const float* temperature, const Layer& proj,
                                     long long* w_bstride);

// ---------------------------------------------------------------------------- synthesis nets
enum Op : int { OP_SOP = 0, OP_BOP = 1, OP_HOP = 2 };
enum Comp : int { COMP_Y = 0, COMP_UV = 1 };

struct Param {
    std::vector<int> shape;
    const float* data;
};

enum NetKind : int { NET_SYNTHESIS = 0, NET_LATENT = 1, NET_ANALYSIS = 2 };

struct Net {
    int kind = NET_SYNTHESIS;
    int op = 0, comp = 0, dtype = DT_F32;
    int chs = 0;           // latent nets: latent channels (160 luma, 96 chroma)
    bool context = false;  // latent nets: a multi-stage context model is present
    int in_ch = 0;         // analysis nets: picture planes in (1 luma, 12 chroma)
    int clip_n[6] = {};    // analysis nets: channels clipped after conv k (0: no clip_thres)
    std::map<std::string, LayerP> L;
    std::map<std::string, float*> vec;  // device f32 vectors (layer norm, temperature)
    size_t vec_bytes = 0;                // device bytes of vec
    size_t device_bytes() const {
        size_t b = vec_bytes;
        for (const auto& kv : L) b += kv.second->dev_bytes;
        return b;
    }
    ~Net();
};
using NetP = std::shared_ptr<Net>;

NetP build_net(Context& ctx, int op, int comp, int dtype, const std::map<std::string, Param>& params);
// `SynthesisPrimary::forward_with`: y_hat -> planar [1][oh][ow] into `out` (f32 plane or
// picture window per PlaneOut).
void primary_forward(Context& ctx, const Net& net, const TensorP& y_hat, int h, int w,
                     const PlaneOut& out);
// `SynthesisSecondary::forward_with`: (luma latent, chroma latent) -> planar [2][oh][ow].
void secondary_forward(Context& ctx, const Net& net, const TensorP& y_luma,
                       const TensorP& y_chroma, int h, int w, const PlaneOut& out);
void primary_out_size(int op, int h, int w, int* oh, int* ow);
void secondary_out_size(int op, int h, int w, int* oh, int* ow);

// ------------------------------------------------------------------- latent reconstruction
// The float networks of `CommonModel::load` (src/model/common.rs:117-129) for component comp
// (160 / 96 latent channels): the hyper-decoder and, when the checkpoint holds one, the
// multi-stage context model.
NetP build_latent_net(Context& ctx, int comp, int dtype, const std::map<std::string, Param>& params);
// `HyperDecoder::forward_with` (src/model/hyper_decoder.rs:58-89): z (NHWC, C channels) -> psi
// (NHWC, 4C channels, out_h x out_w).
TensorP hyper_decoder_forward(Context& ctx, const Net& net, const TensorP& z, int out_h, int out_w);
// `ContextModel::decompress_with` (src/model/mcm.rs:171-240), or for a net without a context
// model the up-shuffled psi plus the residual (src/decoder/reconstruct.rs:191-202), for psi->n
// regions of one shape at once: residual planar f32 on the device ([C] planes with the given row
// / plane strides; item b's H x W window starts at (rwin.x0[b], rwin.y0[b])) and psi (NHWC, 4C,
// ceil(H/2) x ceil(W/2) per item) -> y_hat planar f32 [N][C][H][W] on the device.
void latent_decompress(Context& ctx, const Net& net, const float* res, long long res_row, long long res_plane,
                       const Windows& rwin, int H, int W, const TensorP& psi, float* y_hat);

// ------------------------------------------------------------------- analysis transforms
// `AnalysisPrimary::load` / `AnalysisSecondary::load` (src/model/analysis.rs:230-290), BOP or HOP.
NetP build_analysis_net(Context& ctx, int op, int comp, int dtype, const std::map<std::string, Param>& params);
// `forward_clip` (src/model/analysis.rs:157-207, :248-310): planar f32 picture planes on the
// device ([in_ch][h][w] in [0, 255]) -> the latent (NHWC, chs channels, h / 16 or h / 8).
TensorP analysis_forward(Context& ctx, const Net& net, const float* x, int h, int w, bool clip);

// Region geometry (src/tools/regions.rs:47-150).
enum RegionPlane : int { PLANE_LATENT = 0, PLANE_PSI = 1, PLANE_HYPER_LATENT = 2, PLANE_IMAGE = 3 };
struct RegionParams {
    bool partitioned = false, independent = false;
    int num_ver = 1, num_hor = 1;
    int hyper_decoder_overlap = 0, mcm_overlap = 0;  // signalled values
};
struct RArea {
    int x = 0, y = 0, w = 0, h = 0;
};
struct RegionGrid {
    int rows = 1, cols = 1;
    std::vector<RArea> core, extended;
};
// `region_grid(hdr, ccs, plane)` of a height x width picture (luma samples).
RegionGrid region_grid(int height, int width, int ccs, const RegionParams& r, int plane);
// `reconstruct_latent` (src/decoder/reconstruct.rs:81-234) of the net's component: host z_hat
// int8 [C][zh][zw] and dequantised residual f32 [C][H][W] -> host psi f32
// [4C][ceil(H/2)][ceil(W/2)] and y_hat f32 [C][H][W] (synchronises).
void reconstruct_latent(Context& ctx, const Net& net, int height, int width, const RegionParams& r,
                        const int8_t* z_hat, int zh, int zw, const float* residual, int H, int W,
                        float* psi, float* y_hat);

}  // namespace zjai
