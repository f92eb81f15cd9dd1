/*
 * zjai_hip.h -- C-ABI of the MI355X (gfx950) synthesis backend for zenjpegai.
 *
 * This is the drop-in boundary a `zenjpegai-hip` Rust crate binds (all `unsafe` stays in that
 * crate; the main crate keeps `#![forbid(unsafe_code)]`). Plain pointers and sizes only.
 *
 * Conventions
 *  - Every entry point returns an int32 status: ZJAI_OK (0) or a negative ZJAI_E_* code. The
 *    codes map 1:1 to `zenjpegai::Error` variants (reference src/error.rs:8-33) plus a device
 *    class; as with the reference's wgpu backend (gpu/src/error.rs:6-25), any failure other than
 *    ZJAI_E_INVALID_ARGUMENT on a well-formed call means "fall back to the CPU engine".
 *    zjai_last_error() returns the message of the context's last failure.
 *  - Host tensors are planar float32 [c][h][w] (the reference's `Tensor<f32>`, src/tensor.rs:12).
 *  - Weights use PyTorch layouts: conv [out][in/groups][kh][kw], transposed conv
 *    [in][out][k][k] (src/nn/mod.rs:56-136). They are copied at creation; host buffers stay
 *    the caller's. Device tensors are NHWC, owned by the context's pool.
 *  - A context owns one HIP stream on one device and must be used by one host thread at a time
 *    (the Rust side holds it behind a Mutex, as `GpuDecoder.workspace`, gpu/src/decoder.rs:212).
 */
#ifndef ZJAI_HIP_H
#define ZJAI_HIP_H

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define ZJAI_API __attribute__((visibility("default")))
#else
#define ZJAI_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define ZJAI_OK 0
#define ZJAI_E_INVALID_ARGUMENT (-1) /* Error::InvalidArgument */
#define ZJAI_E_UNSUPPORTED (-2)      /* Error::Unsupported */
#define ZJAI_E_LIMIT (-3)            /* Error::LimitExceeded (device memory) */
#define ZJAI_E_MODEL (-4)            /* Error::Model (bad weight shapes / missing tensors) */
#define ZJAI_E_CANCELLED (-5)        /* Error::Cancelled */
#define ZJAI_E_DEVICE (-6)           /* HIP runtime / device failure */

/* Precision of a layer / net: storage type of weights and activations. Accumulation is f32. */
#define ZJAI_F32 0  /* fp32 MFMA parity path */
#define ZJAI_F16 1  /* f16 inputs, fp32 accumulate */
#define ZJAI_BF16 2 /* bf16 inputs, fp32 accumulate */

/* Operating points and components (reference src/header.rs:39, src/model/synthesis.rs). */
#define ZJAI_OP_SOP 0
#define ZJAI_OP_BOP 1
#define ZJAI_OP_HOP 2
#define ZJAI_COMP_Y 0
#define ZJAI_COMP_UV 1

/* Fused epilogue selectors (zjai_conv_forward_fused). */
#define ZJAI_ACT_NONE 0
#define ZJAI_ACT_RELU 1
#define ZJAI_ACT_LEAKY_RELU 2
#define ZJAI_ACT_SIGMOID 3
#define ZJAI_RES_NONE 0
#define ZJAI_RES_ADD 1  /* y = a + r1 */
#define ZJAI_RES_GATE 2 /* y = r1 * (1 + a) */
#define ZJAI_RES_CAB 3  /* y = r1 * sigmoid(a) + r2 */
#define ZJAI_RES_MUL 4  /* y = r1 * a */

typedef struct zjai_ctx zjai_ctx;
typedef struct zjai_tensor zjai_tensor;
typedef struct zjai_layer zjai_layer;
typedef struct zjai_net zjai_net;
typedef struct zjai_picture zjai_picture;

/* ------------------------------------------------------------------ context / diagnostics */

/* Replaces `Engine` construction (src/nn/fast/mod.rs:128-172) for the HIP backend: binds a
 * device and creates its stream. flags: 0 or an OR of ZJAI_CTX_UNFUSED_BLOCKS,
 * ZJAI_CTX_PHASE_SPLIT_CONVT, ZJAI_CTX_MFMA16_CONV3X3, ZJAI_CTX_IGEMM_CONV1X1,
 * ZJAI_CTX_COUNT_F16_RANGE and ZJAI_CTX_VALU_NARROW_CONVT (other bits are rejected). */
/* Run the transformer blocks (src/model/attention.rs:328-372) as the reference's separate ops --
 * layer norm, 1x1, depthwise (+ ELU gate), 1x1 -- instead of the fused kernels every precision
 * uses by default for `prep_data` (LN + 1x1 + depthwise) and for the feed-forward half, and the
 * 32- / 64-channel ResAUs (src/model/synthesis.rs:24-74) as their grouped 3x3 and gated 1x1
 * instead of one fused kernel (each pair gives bit-identical results). */
#define ZJAI_CTX_UNFUSED_BLOCKS 0x1u
/* Run every 3x3 stride-2 transposed convolution (`conv3x3_t`, src/model/attention.rs:78-91) one
 * output phase per workgroup. By default a layer whose four-phase grid fills the chip (>= 256
 * workgroups) runs all four phases per workgroup and a smaller one runs phase-split on a narrow
 * tile (same results bit for bit; the flag is for A/B runs and the parity test that proves it). */
#define ZJAI_CTX_PHASE_SPLIT_CONVT 0x2u
/* Run the dense stride-1 3x3 convolutions of the 16-bit precisions on the 16x16x32 MFMA kernel
 * instead of the 32x32x16 one (for A/B runs and the test that compares the two). */
#define ZJAI_CTX_MFMA16_CONV3X3 0x4u
/* Run the 1x1 convolutions on the implicit-GEMM conv kernel instead of the dedicated 1x1 GEMM
 * kernel (same results bit for bit; for A/B runs and the test that proves it). */
#define ZJAI_CTX_IGEMM_CONV1X1 0x8u
/* Count the f16 activations the context's kernels store as non-finite: an IEEE overflow (a
 * value whose rounding exceeds 65504 is stored as +-inf) or a NaN. After every launch that writes
 * an f16 tensor a scan adds the tensor's non-finite samples to a device counter, read by
 * zjai_get_stats (`f16_nonfinite`). No counterpart in the reference (its f16 study rounds
 * weights only, src/weights/f16.rs:70-72, with f32 activations); it tells whether a 16-bit run of
 * a net stayed inside f16's range. Off by default: one extra pass over every f16 tensor. */
#define ZJAI_CTX_COUNT_F16_RANGE 0x10u
/* Run the f16 / bf16 3x3 stride-2 transposed convolutions with at most 8 outputs (the last
 * synthesis layers) on the vector ALUs in the reference's (input channel, tap) FMA order
 * instead of the matrix cores. The MFMA form sums the same exact products in another order, so
 * the two differ by the summation order before the final rounding to the storage type; the fp32
 * path always uses the vector form (bit-exact against the oracle). For A/B runs and the tests
 * that compare the two. */
#define ZJAI_CTX_VALU_NARROW_CONVT 0x20u
ZJAI_API int32_t zjai_ctx_create(int32_t device, uint32_t flags, zjai_ctx** out);
ZJAI_API int32_t zjai_ctx_destroy(zjai_ctx* ctx);
/* Copies the last failure message (NUL-terminated, truncated to len). Works with ctx == NULL
 * for failures of zjai_ctx_create. */
ZJAI_API int32_t zjai_last_error(const zjai_ctx* ctx, char* buf, size_t len);
/* Blocks until the context's stream is idle. */
ZJAI_API int32_t zjai_sync(zjai_ctx* ctx);
/* Cooperative cancellation, the `enough::Stop` check between layers and tiles
 * (src/decoder/api.rs:283-299): while set, running calls return ZJAI_E_CANCELLED at their next
 * check. */
ZJAI_API int32_t zjai_set_stop(zjai_ctx* ctx, int32_t stop);

typedef struct zjai_stats {
    float last_run_ms;        /* device time of the last zjai_picture_run (HIP events) */
    int64_t kernel_launches;  /* launches issued by the context so far */
    uint64_t pool_in_use;     /* device bytes held by live tensors */
    uint64_t pool_peak;       /* high-water mark of pool_in_use since the last zjai_release_buffers */
    uint64_t pool_cached;     /* device bytes held by the pools in total (live + cached blocks) */
    uint64_t f16_nonfinite;   /* ZJAI_CTX_COUNT_F16_RANGE: non-finite f16 samples stored so far */
} zjai_stats;
/* Replaces the reference's `DecodeStats` probe (src/decoder/stats.rs:301) for device work. With
 * ZJAI_CTX_COUNT_F16_RANGE it synchronises the context's streams to read the counter. */
ZJAI_API int32_t zjai_get_stats(zjai_ctx* ctx, zjai_stats* out);
/* Host-side failure injection for tests of the error paths. After `after` more successful
 * events of kind `what` the next one fails, once: ZJAI_FAIL_ALLOC counts device pool
 * allocations (cached or not) and fails one as an out-of-memory hipMalloc does
 * (ZJAI_E_LIMIT); ZJAI_FAIL_LAUNCH counts kernel launches and fails one as a failed launch does
 * (ZJAI_E_DEVICE). The failure is raised on the host before the allocation or launch, so nothing
 * faulty reaches the device, and the context stays usable. ZJAI_FAIL_NONE disarms. It exercises
 * the reference GPU backend's rule that such failures mean "fall back to the CPU engine"
 * (gpu/src/error.rs:6-25). */
#define ZJAI_FAIL_NONE 0
#define ZJAI_FAIL_ALLOC 1
#define ZJAI_FAIL_LAUNCH 2
ZJAI_API int32_t zjai_inject_failure(zjai_ctx* ctx, int32_t what, int64_t after);
/* Per-launch profile, the device-side counterpart of the reference's GPU `Timing` / per-dispatch
 * profile (gpu/src/synthesis.rs:758): between begin and end every kernel launch of the context
 * is bracketed by HIP events on its stream. zjai_profile_end synchronises and writes up to `cap`
 * records (kernel name as profilers print it, algorithmic FLOPs and compulsory HBM bytes of the
 * launch, measured milliseconds); *n = number of launches profiled. */
typedef struct zjai_prof_record {
    char name[96];
    double flops;
    double bytes;
    float ms;
} zjai_prof_record;
ZJAI_API int32_t zjai_profile_begin(zjai_ctx* ctx);
ZJAI_API int32_t zjai_profile_end(zjai_ctx* ctx, zjai_prof_record* out, int32_t cap, int32_t* n);
/* Returns cached pool blocks to the device (`release_buffers`, src/nn/fast/tensor.rs:122), the
 * lanes' included, and starts a new pool_peak. The pool figures of zjai_get_stats cover the
 * context's own pool and every lane's (pool_peak: the sum of the pools' high-water marks). */
ZJAI_API int32_t zjai_release_buffers(zjai_ctx* ctx);

/* ----------------------------------------------------------------------- device tensors */

/* `BTensor::zeros` / `scratch` (src/nn/fast/tensor.rs:203-230) on the device: [c][h][w] stored
 * NHWC with the channel stride padded to 8. */
ZJAI_API int32_t zjai_tensor_create(zjai_ctx* ctx, int32_t c, int32_t h, int32_t w, int32_t precision,
                           zjai_tensor** out);
/* `BTensor::from_planar` (src/nn/fast/tensor.rs:251): host planar f32 [c][h][w] -> new device
 * tensor. */
ZJAI_API int32_t zjai_tensor_from_planar(zjai_ctx* ctx, const float* data, int32_t c, int32_t h,
                                int32_t w, int32_t precision, zjai_tensor** out);
/* `BTensor::to_planar` (src/nn/fast/tensor.rs:265): device tensor -> host planar f32
 * (capacity `len` floats; needs c*h*w). Synchronises the stream. */
ZJAI_API int32_t zjai_tensor_to_planar(zjai_ctx* ctx, const zjai_tensor* t, float* data, size_t len);
ZJAI_API int32_t zjai_tensor_shape(const zjai_tensor* t, int32_t* c, int32_t* h, int32_t* w,
                          int32_t* precision);
/* `BTensor::crop_par` (src/nn/fast/tensor.rs:349): top-left h x w view (shares storage). */
ZJAI_API int32_t zjai_tensor_crop(zjai_ctx* ctx, const zjai_tensor* t, int32_t h, int32_t w,
                         zjai_tensor** out);
/* `BTensor::cat` (src/nn/fast/tensor.rs:402): channel concatenation into a new tensor. */
ZJAI_API int32_t zjai_tensor_cat(zjai_ctx* ctx, const zjai_tensor* const* parts, int32_t n,
                        zjai_tensor** out);
ZJAI_API int32_t zjai_tensor_destroy(zjai_tensor* t);

/* ------------------------------------------------------------------------------- layers */

/* `ConvLayer::with_extra_pad(Conv2d, &Engine, extra_pad)` (src/nn/fast/layers.rs:36) /
 * `PackedConv::new` (src/nn/fast/conv.rs:524) and `PackedDepthwise::new`
 * (src/nn/fast/depthwise.rs:103): weight [out][in/groups][kh][kw], bias nullable,
 * extra_pad [top, left, bottom, right] or NULL. Supported: 1x1, 2x2, 3x3 stride 1; 3x3
 * stride 2; depthwise 3x3. Other geometries return ZJAI_E_UNSUPPORTED. */
ZJAI_API int32_t zjai_conv2d_create(zjai_ctx* ctx, int32_t in_ch, int32_t out_ch, int32_t kh, int32_t kw,
                           int32_t stride, int32_t pad_h, int32_t pad_w, int32_t groups,
                           const float* weight, const float* bias, const int32_t* extra_pad,
                           int32_t precision, zjai_layer** out);
/* `ConvTransposeLayer::new(ConvTranspose2d)` (src/nn/fast/layers.rs:136) /
 * `PackedConvTranspose::new` (src/nn/fast/conv.rs:1919): weight [in][out][k][k]; stride 2
 * with k in {3, 4}. */
ZJAI_API int32_t zjai_conv_transpose2d_create(zjai_ctx* ctx, int32_t in_ch, int32_t out_ch, int32_t k,
                                     int32_t stride, int32_t pad, int32_t out_pad,
                                     const float* weight, const float* bias, int32_t precision,
                                     zjai_layer** out);
ZJAI_API int32_t zjai_layer_destroy(zjai_layer* layer);
/* `ConvLayer::forward` / `ConvTransposeLayer::forward` (src/nn/fast/layers.rs:92, :162):
 * new output tensor. */
ZJAI_API int32_t zjai_conv_forward(zjai_ctx* ctx, const zjai_layer* layer, const zjai_tensor* x,
                          zjai_tensor** out);
/* Forward with a fused epilogue: act (ZJAI_ACT_*), then res (ZJAI_RES_*) against r1 / r2
 * (tensors with the output's shape), optional pixel shuffle r (1 = none) and relu6 applied
 * to x on load. Equals the reference's layer followed by its elementwise ops
 * (src/nn/fast/layers.rs:174-289, src/nn/fast/math.rs:371-397). */
ZJAI_API int32_t zjai_conv_forward_fused(zjai_ctx* ctx, const zjai_layer* layer, const zjai_tensor* x,
                                int32_t act, int32_t res, const zjai_tensor* r1,
                                const zjai_tensor* r2, int32_t pixel_shuffle,
                                int32_t relu6_input, zjai_tensor** out);

/* ------------------------------------------------------------------- elementwise (in place) */
/* src/nn/fast/layers.rs:204-229, src/model/hyper_encoder.rs:24, src/nn/fast/math.rs:371-397 */
ZJAI_API int32_t zjai_relu(zjai_ctx* ctx, zjai_tensor* x);
ZJAI_API int32_t zjai_relu6(zjai_ctx* ctx, zjai_tensor* x);
ZJAI_API int32_t zjai_leaky_relu(zjai_ctx* ctx, zjai_tensor* x);
ZJAI_API int32_t zjai_sigmoid(zjai_ctx* ctx, zjai_tensor* x);
ZJAI_API int32_t zjai_add_assign(zjai_ctx* ctx, zjai_tensor* dst, const zjai_tensor* src);
ZJAI_API int32_t zjai_gate(zjai_ctx* ctx, zjai_tensor* x, const zjai_tensor* mask);
ZJAI_API int32_t zjai_mul_assign(zjai_ctx* ctx, zjai_tensor* a, const zjai_tensor* b);
ZJAI_API int32_t zjai_elu_gate(zjai_ctx* ctx, zjai_tensor* a, const zjai_tensor* b);
/* `pixel_shuffle(&Engine, &BTensor, r)` (src/nn/fast/layers.rs:262). */
ZJAI_API int32_t zjai_pixel_shuffle(zjai_ctx* ctx, const zjai_tensor* x, int32_t r, zjai_tensor** out);
/* `math::layer_norm_channels` (src/nn/fast/math.rs:423), into a new tensor. */
ZJAI_API int32_t zjai_layer_norm_channels(zjai_ctx* ctx, const zjai_tensor* x, const float* weight,
                                 const float* bias, zjai_tensor** out);
/* `math::channel_attention` (src/nn/fast/math.rs:512): qkv [3*dim] channels -> [dim]. */
ZJAI_API int32_t zjai_channel_attention(zjai_ctx* ctx, const zjai_tensor* qkv, int32_t heads,
                               const float* temperature, zjai_tensor** out);
/* Allocation-free channel attention. It has no counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Same result as zjai_channel_attention, bit for bit. qkv and
 * out are caller-owned device buffers, 16-byte aligned, NHWC dense in `precision`: qkv
 * [h][w][channels] (channels = 3 * dim: q, k, v), out [h][w][dim]; temperature is a device array
 * of `heads` floats. The work is enqueued on the context's stream (zjai_sync waits for it) and
 * allocates nothing: its scratch (Gram partial sums, attention matrix, folded weight) is one
 * static device array of ZJAI_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends and
 * shared by every call on that GPU, so calls that overlap on one GPU (contexts on different
 * streams) race. A map that needs more scratch (with dim 128 and 4 heads: more than ~240k
 * positions) returns ZJAI_E_LIMIT before anything is launched. */
#define ZJAI_NOALLOC_SCRATCH_BYTES (16u << 20)
ZJAI_API int32_t zjai_channel_attention_noalloc(zjai_ctx* ctx, const void* qkv, int32_t channels,
                                                int32_t h, int32_t w, int32_t heads,
                                                const float* temperature, int32_t precision,
                                                void* out);

/* ------------------------------------------------------------------------ synthesis nets */

/* `SynthesisPrimary::load` / `SynthesisSecondary::load` (src/model/synthesis.rs:242, :972) from
 * named checkpoint tensors (names and shapes of fuzz/fuzz_targets/common.rs:260-345, e.g.
 * "first_stage.0.0.conv1.weight"). shapes: ndims[i] dims each, concatenated in `dims`. */
ZJAI_API int32_t zjai_net_create(zjai_ctx* ctx, int32_t op, int32_t component, int32_t precision,
                        int32_t n_tensors, const char* const* names, const int32_t* ndims,
                        const int32_t* dims, const float* const* data, zjai_net** out);
ZJAI_API int32_t zjai_net_destroy(zjai_net* net);
/* Output plane size of a net for an h x w target (>= h x w; the caller crops). */
ZJAI_API int32_t zjai_net_out_size(const zjai_net* net, int32_t h, int32_t w, int32_t* oh, int32_t* ow);
/* Device bytes a net's packed weights, biases and vectors hold (any net kind). With the
 * estimate of zjai_picture_estimate_memory it sizes a decode's device memory, as the reference's
 * `estimate_memory` counts the packed networks in its fixed term (src/decoder/limits.rs:164). */
ZJAI_API int32_t zjai_net_device_bytes(const zjai_net* net, uint64_t* bytes);
/* `SynthesisPrimary::forward_with` (src/model/synthesis.rs:262): y_hat [160][lh][lw] device
 * tensor -> host planar [1][oh][ow] in [0, 255] (capacity `len` floats). */
ZJAI_API int32_t zjai_primary_forward(zjai_ctx* ctx, const zjai_net* net, const zjai_tensor* y_hat,
                             int32_t h, int32_t w, float* out, size_t len);
/* `SynthesisSecondary::forward_with` (src/model/synthesis.rs:1004): luma [160] and chroma [96]
 * latents -> host planar [2][oh][ow] in [0, 255]. */
ZJAI_API int32_t zjai_secondary_forward(zjai_ctx* ctx, const zjai_net* net, const zjai_tensor* y_luma,
                               const zjai_tensor* y_chroma, int32_t h, int32_t w, float* out,
                               size_t len);

/* ----------------------------------------------------------------------- picture driver */

/* One synthesis tile (reference `SynthesisTile`, src/tools/tiles.rs:26-35). */
typedef struct zjai_tile {
    int32_t image_x, image_y, image_w, image_h;
    int32_t latent_x, latent_y, latent_w, latent_h;
    int32_t core_x, core_y, core_w, core_h;
    int32_t core_off_x, core_off_y;
} zjai_tile;

/* Tile layout of a height x width picture (`synthesis_tiles`, src/tools/tiles.rs:39-119).
 * tile_size == 0 disables tiling. With region_rows/cols > 0 tiles respect that grid of
 * independent regions (`region_grid(hdr, 0, Plane::Image)`, src/tools/regions.rs:116-150).
 * Writes up to `cap` tiles, *n = count (ZJAI_E_LIMIT if cap is too small). */
ZJAI_API int32_t zjai_synthesis_tiles(int32_t height, int32_t width, int32_t latent_h, int32_t latent_w,
                             int32_t tile_size, int32_t overlap, int32_t region_rows,
                             int32_t region_cols, zjai_tile* tiles, int32_t cap, int32_t* n);

/* The synthesis half of `reconstruct::synthesize_with` (src/decoder/reconstruct.rs:285-331) plus
 * `quantize_plane` (src/decoder/output.rs:330): plans a picture of height x width from latents
 * [160][lh][lw] (+ [96][lh][lw] when net_uv is given), tiles as given, chroma subsampling
 * sv x sh, displayed size out_h x out_w, output bit depth (0 = float planes in [0, 255]). */
ZJAI_API int32_t zjai_picture_create(zjai_ctx* ctx, const zjai_net* net_y, const zjai_net* net_uv,
                            int32_t lh, int32_t lw, int32_t height, int32_t width,
                            const zjai_tile* tiles, int32_t n_tiles, int32_t sv, int32_t sh,
                            int32_t out_h, int32_t out_w, int32_t bit_depth, zjai_picture** out);
ZJAI_API int32_t zjai_picture_destroy(zjai_picture* pic);
/* Uploads the decoded latents once (planar f32; uv_hat may be NULL without net_uv). */
ZJAI_API int32_t zjai_picture_upload(zjai_ctx* ctx, zjai_picture* pic, const float* y_hat,
                            const float* uv_hat);
/* Device memory of one picture before anything is allocated, the counterpart of the reference's
 * `estimate_memory` (src/decoder/limits.rs:164-245; host only, no device needed). Arguments as
 * zjai_picture_create's, with the nets given by operating point, precision and whether a chroma
 * net runs, and the lane count of zjai_picture_set_lanes. Figures:
 *   picture_bytes: the latents and output planes zjai_picture_create allocates (exact);
 *   live_bytes: the buffer-pool blocks the tile batches hold at once (lanes run together), the
 *     decode's working set (the reference's `live_bytes`);
 *   pool_bytes: the blocks the pools keep cached after the run on a released context
 *     (zjai_release_buffers returns them; a pool also frees them and retries when the device runs
 *     out), >= live_bytes.
 * live and pool are models calibrated on measured pool use that bound it from above (bytes per
 * sample of each tile batch's 16 x latent window, +8 %). The nets' own bytes
 * (zjai_net_device_bytes) and the buffers of zjai_picture_download_rgb (6 bytes per displayed
 * pixel, 18 with float planes) are not included. */
typedef struct zjai_memory_estimate {
    uint64_t picture_bytes;
    uint64_t live_bytes;
    uint64_t pool_bytes;
} zjai_memory_estimate;
ZJAI_API int32_t zjai_picture_estimate_memory(int32_t op, int32_t precision, int32_t with_uv, int32_t lh,
                                              int32_t lw, int32_t height, int32_t width,
                                              const zjai_tile* tiles, int32_t n_tiles, int32_t sv,
                                              int32_t sh, int32_t out_h, int32_t out_w, int32_t bit_depth,
                                              int32_t lanes, zjai_memory_estimate* out);
/* Admission bound (`Limits::max_memory_bytes`, src/decoder/limits.rs:30-34, checked by
 * `check_header` :106-111): with bytes > 0, zjai_picture_create and zjai_picture_set_lanes refuse
 * with ZJAI_E_LIMIT, before allocating anything, a picture whose nets (zjai_net_device_bytes)
 * plus picture_bytes and live_bytes of zjai_picture_estimate_memory at its lane count exceed
 * `bytes`. 0 (the default) disables the check. */
ZJAI_API int32_t zjai_ctx_set_memory_limit(zjai_ctx* ctx, uint64_t bytes);
/* Runs every tile, on the context's stream or spread over lanes (see zjai_picture_set_lanes),
 * and waits for the picture (latents must be uploaded). */
ZJAI_API int32_t zjai_picture_run(zjai_ctx* ctx, zjai_picture* pic);
/* Runs the picture's tile batches on `lanes` (1..8) concurrent streams of the context, each with
 * its own buffer pool; 1 (the default) keeps everything on the context's stream. Mirrors the
 * reference's tile-parallel synthesis (rayon over tiles, src/decoder/reconstruct.rs:379-464):
 * tiles are independent and write disjoint core rectangles. */
ZJAI_API int32_t zjai_picture_set_lanes(zjai_ctx* ctx, zjai_picture* pic, int32_t lanes);
/* Replay mode (on = 1): the next zjai_picture_run captures the picture's whole launch sequence --
 * every tile batch on every lane -- once as a HIP graph instead of issuing it launch by launch,
 * then launches it; later runs launch the same graph again (one host call per picture). Mirrors
 * the reference's GPU backend, which records a dispatch plan per tile geometry and replays it
 * (gpu/src/synthesis.rs:1163-1185, plan built by gpu/src/plan.rs:877 `Graph::finish`). The graph
 * reads the picture's latent buffers and writes its planes, so zjai_picture_upload between runs
 * takes effect; the intermediate buffers it addresses are taken out of the context's pools for
 * its lifetime. Changing the lane count captures again; on = 0 drops the graph and its buffers.
 * Eager and replayed runs give the same bytes. Per-launch profiling must be off while capturing;
 * the stop flag is checked before a replay, not inside it; launch counts (zjai_get_stats) include
 * a replay's launches; injected launch failures (zjai_inject_failure) count launches issued from
 * the host, i.e. eager runs and the capture, not the kernels of a replay. */
ZJAI_API int32_t zjai_picture_set_replay(zjai_ctx* ctx, zjai_picture* pic, int32_t on);
/* Copies the planes out (synchronises): Y out_h*out_w, U/V ceil(out_h/sv)*ceil(out_w/sh)
 * samples each, as float (bit_depth 0) or uint16. u/v may be NULL without net_uv. */
ZJAI_API int32_t zjai_picture_download(zjai_ctx* ctx, zjai_picture* pic, void* y, void* u, void* v);
/* Page-locked host memory (hipHostMalloc) of `bytes` bytes, 16-byte aligned, for the host
 * buffers of zjai_picture_upload / zjai_picture_download and the other copies: the device reads
 * and writes it directly at the link's DMA rate, where pageable memory goes through the
 * runtime's staging copies (config 5 fp32 from latents on the host to planes on the host: 36.6
 * -> 34.8 ms). No counterpart in the reference, whose host buffers are plain `Vec`s
 * (src/nn/fast/tensor.rs); for callers that keep transfer buffers across pictures. Release with
 * zjai_host_free (ctx may be NULL there: the memory outlives the context); bytes == 0 is an
 * error. */
ZJAI_API int32_t zjai_host_alloc(zjai_ctx* ctx, size_t bytes, void** out);
ZJAI_API int32_t zjai_host_free(zjai_ctx* ctx, void* p);

/* ------------------------------------------------------------------------ output stage */

#define ZJAI_RESIZE_BICUBIC 0  /* decoder::output::resize_bicubic (src/decoder/output.rs:117) */
#define ZJAI_RESIZE_BILINEAR 1 /* nn::resize_bilinear (src/nn/resample.rs:43) */

/* `F.interpolate(x, (out_h, out_w), mode, align_corners=True)` with PyTorch's CPU arithmetic, as
 * the reference restates it (the resamplers behind `Image.to_444_` / `to_420_` / `to_422_`):
 * host planar [c][h][w] f32 -> host planar [c][out_h][out_w] f32 (synchronises). Empty input
 * sizes are ZJAI_E_INVALID_ARGUMENT, like the reference. */
ZJAI_API int32_t zjai_resize(zjai_ctx* ctx, int32_t mode, const float* src, int32_t c, int32_t h,
                             int32_t w, int32_t out_h, int32_t out_w, float* dst);
/* The decoder's output stage for a BT.709 stream on the device: `to_source_format`
 * (src/decoder/output.rs:153-199, chroma bicubic to 4:4:4) then `finish` (:346-366:
 * `to_rgb_planes`, clip, `quantize` with round half to even) over a picture run with float
 * planes (bit_depth 0 at zjai_picture_create) and a chroma net. Writes interleaved RGB
 * uint16 [out_h][out_w][3] at bit_depth 8 or 10 and, when rgb_planes is not NULL, the float
 * planes [3][out_h][out_w] in [0, 255] (the reference's `RgbPlanes`). Synchronises. */
ZJAI_API int32_t zjai_picture_download_rgb(zjai_ctx* ctx, zjai_picture* pic, int32_t bit_depth,
                                           uint16_t* rgb, float* rgb_planes);

/* ----------------------------------------------------------------- latent reconstruction */

/* Region partitioning of a picture header (`Regions`, src/header.rs; the grid of
 * src/tools/regions.rs:104-150). A NULL zjai_regions* means "not partitioned". */
typedef struct zjai_regions {
    int32_t num_ver, num_hor;        /* region rows / columns (>= 1) */
    int32_t independent;             /* independent regions: no overlap extension */
    int32_t hyper_decoder_overlap;   /* signalled value (HyperDecoderOverlap = 2 x this) */
    int32_t mcm_overlap;             /* signalled value (McmOverlap = 4 x this) */
} zjai_regions;

typedef struct zjai_area {
    int32_t x, y, width, height;
} zjai_area;

#define ZJAI_PLANE_LATENT 0       /* y, 1/16 of luma (`Plane::Latent`) */
#define ZJAI_PLANE_PSI 1          /* hyper-decoder output, 1/32 (`Plane::Psi`) */
#define ZJAI_PLANE_HYPER_LATENT 2 /* z, 1/64 (`Plane::HyperLatent`) */
#define ZJAI_PLANE_IMAGE 3        /* the picture in luma samples (`Plane::Image`) */

/* `region_grid(hdr, ccs, plane)` (src/tools/regions.rs:116-150) of a height x width picture for
 * component 0 (luma) or 1 (chroma): writes up to `cap` core and extended areas (row-major),
 * *n = count (ZJAI_E_LIMIT if cap is too small). Host only; needs no context. */
ZJAI_API int32_t zjai_region_grid(int32_t height, int32_t width, int32_t component,
                                  const zjai_regions* regions, int32_t plane, zjai_area* core,
                                  zjai_area* extended, int32_t cap, int32_t* n);

/* The float networks of `CommonModel::load` (src/model/common.rs:117-129) for component 0 / 1
 * (160 / 96 latent channels) from named checkpoint tensors: `HyperDecoder::load`
 * (src/model/hyper_decoder.rs:24-45, "hyper_decoder.conv1..4") and, when
 * "context.MCM.0.fusion_pred_net.conv1.weight" is present, `ContextModel::load`
 * (src/model/mcm.rs:123-159, "context.MCM.{0..3}.{conv.0,conv.1,fusion_pred_net.conv1..3}"). */
ZJAI_API int32_t zjai_latent_model_create(zjai_ctx* ctx, int32_t component, int32_t precision,
                                          int32_t n_tensors, const char* const* names,
                                          const int32_t* ndims, const int32_t* dims,
                                          const float* const* data, zjai_net** out);
/* Latent channels of the model and whether it holds a context model. */
ZJAI_API int32_t zjai_latent_model_info(const zjai_net* net, int32_t* channels, int32_t* has_context);
/* `HyperDecoder::forward` (src/model/hyper_decoder.rs:47-89): z_hat int8 [c][zh][zw] -> psi
 * f32 [4c][out_h][out_w] on the host (the 2x upsampled map cropped to out_h x out_w). */
ZJAI_API int32_t zjai_hyper_decoder_forward(zjai_ctx* ctx, const zjai_net* net, const int8_t* z_hat,
                                            int32_t c, int32_t zh, int32_t zw, int32_t out_h,
                                            int32_t out_w, float* psi, size_t len);
/* `ContextModel::decompress` (src/model/mcm.rs:161-240): dequantised residual f32 [c][h][w] and
 * psi f32 [4c][psi_h][psi_w] (psi_h = ceil(h/2), psi_w = ceil(w/2)) -> y_hat f32 [c][h][w].
 * A model without a context model returns the up-shuffled psi plus the residual instead
 * (src/decoder/reconstruct.rs:191-202, `upshuffle_psi_par` src/model/mcm.rs:742). */
ZJAI_API int32_t zjai_context_decompress(zjai_ctx* ctx, const zjai_net* net, const float* residual,
                                         int32_t c, int32_t h, int32_t w, const float* psi,
                                         int32_t psi_h, int32_t psi_w, float* y_hat, size_t len);
/* `reconstruct::reconstruct_latent` (src/decoder/reconstruct.rs:81-234) for the model's
 * component of a height x width picture: hyper-decoder per region on its z window, psi merged
 * in raster order, context model per region on its residual / psi windows, y_hat merged (whole
 * latent areas for independent regions, one sample dropped per interior side otherwise).
 * z_hat int8 [c][zh][zw], residual f32 [c][h][w] -> psi f32 [4c][ceil(h/2)][ceil(w/2)] and y_hat
 * f32 [c][h][w] on the host (synchronises). */
ZJAI_API int32_t zjai_reconstruct_latent(zjai_ctx* ctx, const zjai_net* net, int32_t height,
                                         int32_t width, const zjai_regions* regions,
                                         const int8_t* z_hat, int32_t zh, int32_t zw,
                                         const float* residual, int32_t h, int32_t w, float* psi,
                                         float* y_hat);

/* ------------------------------------------------------------------------- weight readers */

/* Host only (no context, no device). Failures return ZJAI_E_MODEL (malformed file, missing or
 * mistyped tensor), ZJAI_E_LIMIT (table sizes, small output buffers) or
 * ZJAI_E_INVALID_ARGUMENT; zjai_last_error(NULL, ...) holds the message. */
typedef struct zjai_checkpoint zjai_checkpoint;
typedef struct zjai_bundle zjai_bundle;

/* Element types by their ZJM1 codes (`dtype_code`, src/weights/packed.rs:62-75). */
#define ZJAI_DTYPE_F64 0
#define ZJAI_DTYPE_F32 1
#define ZJAI_DTYPE_F16 2
#define ZJAI_DTYPE_I64 3
#define ZJAI_DTYPE_I32 4
#define ZJAI_DTYPE_I16 5
#define ZJAI_DTYPE_I8 6
#define ZJAI_DTYPE_U8 7
#define ZJAI_DTYPE_BOOL 8
#define ZJAI_MAX_RANK 8

/* `Checkpoint::parse` (src/weights/mod.rs:135-187): a packed ZJM1 file (by its magic) or a
 * PyTorch `.pth` checkpoint (stored ZIP, `src/weights/zip.rs`, whose data.pkl runs through a
 * data-only pickle interpreter, `src/weights/pickle.rs`: nothing in the file is executed).
 * The bytes are copied; the caller may free them on return. */
ZJAI_API int32_t zjai_checkpoint_parse(const void* data, size_t len, zjai_checkpoint** out);
ZJAI_API int32_t zjai_checkpoint_destroy(zjai_checkpoint* ck);
/* Top-level tensors (nested dict leaves as dotted names), integer entries and numeric lists
 * (`tensor_names`, `ints`, `list`, src/weights/mod.rs:189-233); packed = 1 for ZJM1. */
ZJAI_API int32_t zjai_checkpoint_counts(const zjai_checkpoint* ck, int32_t* tensors, int32_t* ints,
                                        int32_t* lists, int32_t* packed);
/* Name of tensor i (file order) into buf (NUL-terminated; ZJAI_E_LIMIT if cap is too small). */
ZJAI_API int32_t zjai_checkpoint_tensor_name(const zjai_checkpoint* ck, int32_t i, char* buf, size_t cap);
/* `Checkpoint::info` (src/weights/mod.rs:198-204): dtype, rank and up to ZJAI_MAX_RANK dims. */
ZJAI_API int32_t zjai_checkpoint_info(const zjai_checkpoint* ck, const char* name, int32_t* dtype,
                                      int32_t* rank, int64_t* shape);
/* `Checkpoint::raw` (src/weights/mod.rs:330-340): contiguous little-endian row-major bytes of
 * any dtype (strided views gathered); `bytes` must equal numel x element size. */
ZJAI_API int32_t zjai_checkpoint_read(const zjai_checkpoint* ck, const char* name, void* out, size_t bytes);
/* `Checkpoint::f32` (src/weights/mod.rs:342-378): an f32 tensor, or an f16 one (ZJB2 members)
 * upcast exactly; `len` must equal numel. */
ZJAI_API int32_t zjai_checkpoint_read_f32(const zjai_checkpoint* ck, const char* name, float* out, size_t len);
/* Integer entry i (`epoch`, ...) and numeric list i (`clip_thres.E1B.MinList`): name into buf;
 * for a list, *n = its length and up to `cap_values` values. */
ZJAI_API int32_t zjai_checkpoint_int_at(const zjai_checkpoint* ck, int32_t i, char* buf, size_t cap,
                                        int64_t* value);
ZJAI_API int32_t zjai_checkpoint_list_at(const zjai_checkpoint* ck, int32_t i, char* buf, size_t cap,
                                         double* values, size_t cap_values, size_t* n);
/* `write_zjm` / `write_zjm_f16` (src/weights/packed.rs:166-225): the named tensors and all
 * integer entries as a ZJM1 file; f16 != 0 stores f32 tensors (except `vr_vec.c`) as f16,
 * round to nearest even. *len = the file size; out == NULL only queries it. */
ZJAI_API int32_t zjai_checkpoint_write_zjm(const zjai_checkpoint* ck, const char* const* names, int32_t n,
                                           int32_t f16, void* out, size_t cap, size_t* len);

/* `PackedBundle::parse` / `add` (src/weights/packed.rs:299-345): ZJB1 / ZJB2 bundles of files
 * addressed by their path relative to the model directory ("VM_common_int/Y_0.012.pth"); a
 * path already present keeps its first copy. The bytes are copied. */
ZJAI_API int32_t zjai_bundle_parse(const void* data, size_t len, zjai_bundle** out);
ZJAI_API int32_t zjai_bundle_add(zjai_bundle* b, const void* data, size_t len);
ZJAI_API int32_t zjai_bundle_destroy(zjai_bundle* b);
/* `paths` (src/weights/packed.rs:347-351): count, then path i into buf. */
ZJAI_API int32_t zjai_bundle_count(const zjai_bundle* b, int32_t* n);
ZJAI_API int32_t zjai_bundle_path(const zjai_bundle* b, int32_t i, char* buf, size_t cap);
/* `ModelSource::read` (src/weights/packed.rs:377-383): a file's bytes, borrowed until the bundle
 * is destroyed (ZJAI_E_MODEL when absent). */
ZJAI_API int32_t zjai_bundle_get(const zjai_bundle* b, const char* rel, const void** data, size_t* len);
/* `notice` (src/weights/packed.rs:368-375): the first bundle's notice text; *len = its length. */
ZJAI_API int32_t zjai_bundle_notice(const zjai_bundle* b, char* buf, size_t cap, size_t* len);
/* `write_bundle` / `write_bundle_f16` (src/weights/packed.rs:235-334): n files as a ZJB1 (or,
 * with f16 != 0, ZJB2) bundle. *len = the bundle size; out == NULL only queries it. */
ZJAI_API int32_t zjai_bundle_write(const char* const* paths, const void* const* files, const size_t* sizes,
                                   int32_t n, const char* notice, int32_t f16, void* out, size_t cap,
                                   size_t* len);

/* zjai_net_create / zjai_latent_model_create with the tensors of a parsed checkpoint
 * (`SynthesisPrimary::load(ck, ...)`, src/model/synthesis.rs:242; `CommonModel::load`,
 * src/model/common.rs:117-129): every f32 (or f16) tensor of the checkpoint is offered by name. */
ZJAI_API int32_t zjai_net_create_from_checkpoint(zjai_ctx* ctx, int32_t op, int32_t component,
                                                 int32_t precision, const zjai_checkpoint* ck,
                                                 zjai_net** out);
ZJAI_API int32_t zjai_latent_model_create_from_checkpoint(zjai_ctx* ctx, int32_t component,
                                                          int32_t precision, const zjai_checkpoint* ck,
                                                          zjai_net** out);

/* ------------------------------------------------------------------ analysis transforms */

/* `AnalysisPrimary::load` / `AnalysisSecondary::load` (src/model/analysis.rs:230-240, :282-290):
 * the encoder's picture -> latent transforms for op BOP or HOP (SOP has none:
 * ZJAI_E_INVALID_ARGUMENT) and component 0 (luma) / 1 (chroma), from named checkpoint tensors
 * ("conv1".."conv5", "act1".."act3", HOP's "TAM" and "cab") and the optional 1-D lists
 * "clip_thres.E{k}{B|H}.MinList" / ".MaxList". Destroy with zjai_net_destroy. */
ZJAI_API int32_t zjai_analysis_create(zjai_ctx* ctx, int32_t op, int32_t component, int32_t precision,
                                      int32_t n_tensors, const char* const* names, const int32_t* ndims,
                                      const int32_t* dims, const float* const* data, zjai_net** out);
ZJAI_API int32_t zjai_analysis_create_from_checkpoint(zjai_ctx* ctx, int32_t op, int32_t component,
                                                      int32_t precision, const zjai_checkpoint* ck,
                                                      zjai_net** out);
/* `forward_clip` (src/model/analysis.rs:248-270, :297-310): picture planes f32 [c][h][w] in
 * [0, 255] on the host -- c = 1 (luma) or c = 12 (half the luma resolution: luma
 * pixel-unshuffled by 2, then U and V likewise) -> latent f32 [160][ceil(h/16)][ceil(w/16)]
 * (component 0) or [96][ceil(h/8)][ceil(w/8)] (component 1) on the host (synchronises).
 * clip != 0 applies the clip_thres lists after each conv. */
ZJAI_API int32_t zjai_analysis_forward(zjai_ctx* ctx, const zjai_net* net, const float* x, int32_t c,
                                       int32_t h, int32_t w, int32_t clip, float* y, size_t len);

#ifdef __cplusplus
}
#endif

#endif /* ZJAI_HIP_H */
