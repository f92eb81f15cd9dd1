// The C-ABI (include/zjai_hip.h): handles, error mapping, tiling geometry and the picture
// driver. No exception or abort crosses this boundary.

#include <algorithm>
#include <array>
#include <cmath>
#include <map>
#include <set>
#include <cstring>
#include <mutex>

#include "checkpoint.h"
#include "runtime.h"

using namespace zjai;

struct zjai_ctx {
    Context c;
};
struct zjai_tensor {
    TensorP t;
};
struct zjai_layer {
    LayerP l;
};
struct zjai_net {
    NetP n;
};

namespace {

std::mutex g_err_mu;
std::string g_err;  // failures with no context (zjai_ctx_create)

template <typename F>
int32_t guard(zjai_ctx* ctx, F&& f) {
    try {
        f();
        return ZJAI_OK;
    } catch (const Error& e) {
        if (ctx) ctx->c.last_error = e.what();
        else {
            std::lock_guard<std::mutex> g(g_err_mu);
            g_err = e.what();
        }
        return e.code;
    } catch (const std::bad_alloc&) {
        if (ctx) ctx->c.last_error = "host allocation failed";
        return ZJAI_E_LIMIT;
    } catch (const std::exception& e) {
        if (ctx) ctx->c.last_error = e.what();
        return ZJAI_E_DEVICE;
    }
}

void need(bool ok, const char* msg) {
    if (!ok) throw Error(ZJAI_E_INVALID_ARGUMENT, msg);
}

TensorP planar_upload(Context& c, const float* data, int ch, int h, int w, int dtype) {
    need(data != nullptr, "null data");
    need(ch > 0 && h > 0 && w > 0, "bad shape");
    need(ch % 4 == 0, "channel count must be a multiple of 4");
    need(dtype >= DT_F32 && dtype <= DT_BF16, "precision");
    TensorP t = c.alloc(1, ch, h, w, dtype);
    const size_t n = (size_t)ch * h * w;
    float* stage = (float*)c.pool.alloc(n * 4);
    std::shared_ptr<void> keep(stage, [&c](void* q) { c.pool.release(q); });
    ZJAI_HIP(hipMemcpyAsync(stage, data, n * 4, hipMemcpyHostToDevice, c.stream));
    {
        LaunchScope sc(c, kname("k_planar_to_nhwc", dtype), 0.0, (4.0 + dtype_size(dtype)) * n);
        ZJAI_HIP(launch_planar_to_nhwc(stage, ch, h, w, Windows{}, 1, h, w, t->v, dtype, c.stream));
    }
    ZJAI_HIP(hipStreamSynchronize(c.stream));
    return t;
}

}  // namespace

// ---------------------------------------------------------------- allocation-free scratch
// Scratch of zjai_channel_attention_noalloc: each GPU holds its own copy of this array until the
// process ends. In host code `scratch` is a host-side stand-in, not device memory: the array's
// address on a device comes from hipGetSymbolAddress (scratch_setup, called by zjai_ctx_create
// with that device current) and only that address is passed to kernels.
static __device__ __align__(256) unsigned char scratch[ZJAI_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int SCRATCH_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[SCRATCH_DEVICES] = {};

void scratch_setup(int device) {
    std::lock_guard<std::mutex> g(g_scratch_mu);
    if (device < 0 || device >= SCRATCH_DEVICES) throw Error(ZJAI_E_UNSUPPORTED, "device index beyond the scratch table");
    if (g_scratch_dev[device]) return;
    void* p = nullptr;
    ZJAI_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) throw Error(ZJAI_E_DEVICE, "hipGetSymbolAddress: no address for the scratch array");
    g_scratch_dev[device] = p;
}

unsigned char* scratch_of(int device) {
    std::lock_guard<std::mutex> g(g_scratch_mu);
    return device >= 0 && device < SCRATCH_DEVICES ? (unsigned char*)g_scratch_dev[device] : nullptr;
}

size_t round_up256(size_t n) { return (n + 255) / 256 * 256; }

}  // namespace

// ------------------------------------------------------------------------------- context
extern "C" int32_t zjai_ctx_create(int32_t device, uint32_t flags, zjai_ctx** out) {
    if (!out) return ZJAI_E_INVALID_ARGUMENT;
    *out = nullptr;
    if (flags & ~(ZJAI_CTX_UNFUSED_BLOCKS | ZJAI_CTX_PHASE_SPLIT_CONVT | ZJAI_CTX_MFMA16_CONV3X3 |
                  ZJAI_CTX_IGEMM_CONV1X1 | ZJAI_CTX_COUNT_F16_RANGE | ZJAI_CTX_VALU_NARROW_CONVT))
        return guard(nullptr, [] { throw Error(ZJAI_E_INVALID_ARGUMENT, "zjai_ctx_create: unknown flags"); });
    zjai_ctx* ctx = new (std::nothrow) zjai_ctx();
    if (!ctx) return ZJAI_E_LIMIT;
    const int32_t rc = guard(nullptr, [&] {
        int n = 0;
        hipError_t e = hipGetDeviceCount(&n);
        if (e != hipSuccess || n == 0)
            throw Error(ZJAI_E_DEVICE, std::string("no HIP device: ") + hipGetErrorString(e));
        if (device < 0 || device >= n) throw Error(ZJAI_E_INVALID_ARGUMENT, "device index out of range");
        hipDeviceProp_t prop;
        ZJAI_HIP(hipGetDeviceProperties(&prop, device));
        if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
            throw Error(ZJAI_E_UNSUPPORTED, std::string("kernels are built for gfx950, device is ") + prop.gcnArchName);
        ZJAI_HIP(hipSetDevice(device));
        scratch_setup(device);
        ctx->c.device = device;
        ctx->c.flags = flags;
        ZJAI_HIP(hipStreamCreateWithFlags(&ctx->c.stream, hipStreamNonBlocking));
        ZJAI_HIP(hipEventCreate(&ctx->c.ev0));
        ZJAI_HIP(hipEventCreate(&ctx->c.ev1));
    });
    if (rc != ZJAI_OK) {
        delete ctx;
        return rc;
    }
    *out = ctx;
    return ZJAI_OK;
}

extern "C" int32_t zjai_ctx_destroy(zjai_ctx* ctx) {
    if (!ctx) return ZJAI_OK;
    if (ctx->c.stream) (void)hipStreamSynchronize(ctx->c.stream);
    if (ctx->c.ev0) (void)hipEventDestroy(ctx->c.ev0);
    if (ctx->c.ev1) (void)hipEventDestroy(ctx->c.ev1);
    if (ctx->c.stream) (void)hipStreamDestroy(ctx->c.stream);
    delete ctx;
    return ZJAI_OK;
}

extern "C" int32_t zjai_last_error(const zjai_ctx* ctx, char* buf, size_t len) {
    if (!buf || len == 0) return ZJAI_E_INVALID_ARGUMENT;
    std::string m;
    if (ctx) m = ctx->c.last_error;
    else {
        std::lock_guard<std::mutex> g(g_err_mu);
        m = g_err;
    }
    const size_t n = std::min(len - 1, m.size());
    std::memcpy(buf, m.data(), n);
    buf[n] = 0;
    return ZJAI_OK;
}

extern "C" int32_t zjai_sync(zjai_ctx* ctx) {
    if (!ctx) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] { ZJAI_HIP(hipStreamSynchronize(ctx->c.stream)); });
}

extern "C" int32_t zjai_set_stop(zjai_ctx* ctx, int32_t stop) {
    if (!ctx) return ZJAI_E_INVALID_ARGUMENT;
    ctx->c.stop = stop;
    return ZJAI_OK;
}

extern "C" int32_t zjai_get_stats(zjai_ctx* ctx, zjai_stats* out) {
    if (!ctx || !out) return ZJAI_E_INVALID_ARGUMENT;
    out->last_run_ms = ctx->c.last_ms;
    out->kernel_launches = ctx->c.launches;
    // The root context's pool and every lane's (lanes run at once, so their peaks can coincide).
    out->pool_in_use = ctx->c.pool.in_use();
    out->pool_peak = ctx->c.pool.peak();
    out->pool_cached = ctx->c.pool.cached();
    for (const auto& l : ctx->c.lanes) {
        out->pool_in_use += l->pool.in_use();
        out->pool_peak += l->pool.peak();
        out->pool_cached += l->pool.cached();
    }
    out->f16_nonfinite = 0;
    if (!(ctx->c.flags & ZJAI_CTX_COUNT_F16_RANGE)) return ZJAI_OK;
    return guard(ctx, [&] { out->f16_nonfinite = f16_range_total(ctx->c); });
}

extern "C" int32_t zjai_inject_failure(zjai_ctx* ctx, int32_t what, int64_t after) {
    if (!ctx) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        need(what == ZJAI_FAIL_NONE || what == ZJAI_FAIL_ALLOC || what == ZJAI_FAIL_LAUNCH, "inject: unknown kind");
        need(after >= 0, "inject: negative count");
        ctx->c.faults->what = what == ZJAI_FAIL_ALLOC ? FAULT_ALLOC : what == ZJAI_FAIL_LAUNCH ? FAULT_LAUNCH : FAULT_NONE;
        ctx->c.faults->left = after;
    });
}

extern "C" int32_t zjai_profile_begin(zjai_ctx* ctx) {
    if (!ctx) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        ZJAI_HIP(hipStreamSynchronize(ctx->c.stream));
        ctx->c.prof.clear();
        ctx->c.ev_used = 0;
        ctx->c.profiling = true;
    });
}

extern "C" int32_t zjai_profile_end(zjai_ctx* ctx, zjai_prof_record* out, int32_t cap, int32_t* n) {
    if (!ctx || !n || cap < 0 || (cap && !out)) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        ctx->c.profiling = false;
        ZJAI_HIP(hipStreamSynchronize(ctx->c.stream));
        *n = (int32_t)ctx->c.prof.size();
        for (int32_t i = 0; i < std::min(cap, *n); ++i) {
            const ProfRec& r = ctx->c.prof[i];
            zjai_prof_record& o = out[i];
            std::memset(o.name, 0, sizeof o.name);
            std::strncpy(o.name, r.name.c_str(), sizeof o.name - 1);
            o.flops = r.flops;
            o.bytes = r.bytes;
            ZJAI_HIP(hipEventElapsedTime(&o.ms, r.a, r.b));
        }
        ctx->c.prof.clear();
        ctx->c.ev_used = 0;
    });
}

extern "C" int32_t zjai_release_buffers(zjai_ctx* ctx) {
    if (!ctx) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        ZJAI_HIP(hipStreamSynchronize(ctx->c.stream));
        ctx->c.pool.trim();
        ctx->c.pool.reset_peak();
        for (const auto& l : ctx->c.lanes) {
            ZJAI_HIP(hipStreamSynchronize(l->stream));
            l->pool.trim();
            l->pool.reset_peak();
        }
    });
}

// -------------------------------------------------------------------------------- tensors
extern "C" int32_t zjai_tensor_create(zjai_ctx* ctx, int32_t c, int32_t h, int32_t w,
                                      int32_t precision, zjai_tensor** out) {
    if (!ctx || !out) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        need(precision >= DT_F32 && precision <= DT_BF16, "precision");
        need(c > 0 && h > 0 && w > 0, "bad shape");
        TensorP t = ctx->c.alloc(1, c, h, w, precision);
        ZJAI_HIP(launch_zero(t->v.p, (size_t)t->v.bstride * dtype_size(precision), ctx->c.stream));
        *out = new zjai_tensor{t};
    });
}

extern "C" int32_t zjai_tensor_from_planar(zjai_ctx* ctx, const float* data, int32_t c, int32_t h,
                                           int32_t w, int32_t precision, zjai_tensor** out) {
    if (!ctx || !out) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] { *out = new zjai_tensor{planar_upload(ctx->c, data, c, h, w, precision)}; });
}

extern "C" int32_t zjai_tensor_to_planar(zjai_ctx* ctx, const zjai_tensor* t, float* data, size_t len) {
    if (!ctx || !t || !data) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        const Tensor& x = *t->t;
        const size_t n = (size_t)x.n * x.c * x.h * x.w;
        need(len >= n, "output buffer too small");
        if (n == 0) return;
        float* stage = (float*)ctx->c.pool.alloc(n * 4);
        std::shared_ptr<void> keep(stage, [ctx](void* q) { ctx->c.pool.release(q); });
        {
            LaunchScope sc(ctx->c, kname("k_nhwc_to_planar", x.dtype), 0.0, (4.0 + dtype_size(x.dtype)) * n);
            ZJAI_HIP(launch_nhwc_to_planar(x.v, x.dtype, x.n, x.c, x.h, x.w, stage, ctx->c.stream));
        }
        ZJAI_HIP(hipMemcpyAsync(data, stage, n * 4, hipMemcpyDeviceToHost, ctx->c.stream));
        ZJAI_HIP(hipStreamSynchronize(ctx->c.stream));
    });
}

extern "C" int32_t zjai_tensor_shape(const zjai_tensor* t, int32_t* c, int32_t* h, int32_t* w,
                                     int32_t* precision) {
    if (!t) return ZJAI_E_INVALID_ARGUMENT;
    if (c) *c = t->t->c;
    if (h) *h = t->t->h;
    if (w) *w = t->t->w;
    if (precision) *precision = t->t->dtype;
    return ZJAI_OK;
}

extern "C" int32_t zjai_tensor_crop(zjai_ctx* ctx, const zjai_tensor* t, int32_t h, int32_t w,
                                    zjai_tensor** out) {
    if (!ctx || !t || !out) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] { *out = new zjai_tensor{crop_view(t->t, h, w)}; });
}

extern "C" int32_t zjai_tensor_cat(zjai_ctx* ctx, const zjai_tensor* const* parts, int32_t n,
                                   zjai_tensor** out) {
    if (!ctx || !parts || n <= 0 || !out) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        int c = 0;
        const Tensor& f = *parts[0]->t;
        for (int i = 0; i < n; ++i) {
            const Tensor& p = *parts[i]->t;
            need(p.n == f.n && p.h == f.h && p.w == f.w && p.dtype == f.dtype, "cat: shapes differ");
            need(p.c % 4 == 0, "cat: channel counts must be multiples of 4");
            c += p.c;
        }
        TensorP y = ctx->c.alloc(f.n, c, f.h, f.w, f.dtype);
        int c0 = 0;
        for (int i = 0; i < n; ++i) {
            const Tensor& p = *parts[i]->t;
            LaunchScope sc(ctx->c, kname("k_copy", p.dtype), 0.0, 2.0 * dtype_size(p.dtype) * p.n * p.c * p.h * p.w);
            ZJAI_HIP(launch_copy(p.v, channel_view(y, c0, p.c)->v, p.dtype, p.n, p.c, p.h, p.w, ctx->c.stream));
            c0 += p.c;
        }
        *out = new zjai_tensor{y};
    });
}

extern "C" int32_t zjai_tensor_destroy(zjai_tensor* t) {
    delete t;
    return ZJAI_OK;
}

// --------------------------------------------------------------------------------- layers
extern "C" int32_t zjai_conv2d_create(zjai_ctx* ctx, int32_t in_ch, int32_t out_ch, int32_t kh,
                                      int32_t kw, int32_t stride, int32_t pad_h, int32_t pad_w,
                                      int32_t groups, const float* weight, const float* bias,
                                      const int32_t* extra_pad, int32_t precision, zjai_layer** out) {
    if (!ctx || !out) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        *out = new zjai_layer{make_conv(ctx->c, in_ch, out_ch, kh, kw, stride, pad_h, pad_w, groups, weight,
                                        bias, extra_pad, precision, false)};
    });
}

extern "C" int32_t zjai_conv_transpose2d_create(zjai_ctx* ctx, int32_t in_ch, int32_t out_ch, int32_t k,
                                                int32_t stride, int32_t pad, int32_t out_pad,
                                                const float* weight, const float* bias,
                                                int32_t precision, zjai_layer** out) {
    if (!ctx || !out) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        *out = new zjai_layer{make_conv_transpose(ctx->c, in_ch, out_ch, k, stride, pad, out_pad, weight, bias,
                                                  precision)};
    });
}

extern "C" int32_t zjai_layer_destroy(zjai_layer* layer) {
    delete layer;
    return ZJAI_OK;
}

extern "C" int32_t zjai_conv_forward(zjai_ctx* ctx, const zjai_layer* layer, const zjai_tensor* x,
                                     zjai_tensor** out) {
    if (!ctx || !layer || !x || !out) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] { *out = new zjai_tensor{conv_forward(ctx->c, *layer->l, x->t, Epilogue{})}; });
}

extern "C" int32_t zjai_conv_forward_fused(zjai_ctx* ctx, const zjai_layer* layer, const zjai_tensor* x,
                                           int32_t act, int32_t res, const zjai_tensor* r1,
                                           const zjai_tensor* r2, int32_t pixel_shuffle,
                                           int32_t relu6_input, zjai_tensor** out) {
    if (!ctx || !layer || !x || !out) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        need(act >= ACT_NONE && act <= ACT_SIGMOID, "act");
        need(res >= RES_NONE && res <= RES_MUL, "res");
        Epilogue e;
        e.act = act;
        e.res = res;
        e.r1 = r1 ? r1->t.get() : nullptr;
        e.r2 = r2 ? r2->t.get() : nullptr;
        e.ps = pixel_shuffle <= 0 ? 1 : pixel_shuffle;
        e.relu6_in = relu6_input ? 1 : 0;
        *out = new zjai_tensor{conv_forward(ctx->c, *layer->l, x->t, e)};
    });
}

// ---------------------------------------------------------------------------- elementwise
static int32_t eltwise(zjai_ctx* ctx, int op, zjai_tensor* x, const zjai_tensor* s) {
    if (!ctx || !x) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        const Tensor& a = *x->t;
        if (op >= EL_ADD) {
            need(s != nullptr, "second operand missing");
            const Tensor& b = *s->t;
            need(a.n == b.n && a.c == b.c && a.h == b.h && a.w == b.w && a.dtype == b.dtype, "shapes differ");
        }
        need(a.c % 4 == 0, "channel count must be a multiple of 4");
        LaunchScope sc(ctx->c, kname("k_eltwise", a.dtype), 0.0, (op >= EL_ADD ? 3.0 : 2.0) * dtype_size(a.dtype) * a.c * a.h * a.w);
        ZJAI_HIP(launch_eltwise(op, a.v, s ? s->t->v : a.v, a.dtype, a.n, a.c, a.h, a.w, ctx->c.stream));
    });
}

extern "C" int32_t zjai_relu(zjai_ctx* ctx, zjai_tensor* x) { return eltwise(ctx, EL_RELU, x, nullptr); }
extern "C" int32_t zjai_relu6(zjai_ctx* ctx, zjai_tensor* x) { return eltwise(ctx, EL_RELU6, x, nullptr); }
extern "C" int32_t zjai_leaky_relu(zjai_ctx* ctx, zjai_tensor* x) { return eltwise(ctx, EL_LEAKY, x, nullptr); }
extern "C" int32_t zjai_sigmoid(zjai_ctx* ctx, zjai_tensor* x) { return eltwise(ctx, EL_SIGMOID, x, nullptr); }
extern "C" int32_t zjai_add_assign(zjai_ctx* ctx, zjai_tensor* d, const zjai_tensor* s) { return eltwise(ctx, EL_ADD, d, s); }
extern "C" int32_t zjai_gate(zjai_ctx* ctx, zjai_tensor* x, const zjai_tensor* m) { return eltwise(ctx, EL_GATE, x, m); }
extern "C" int32_t zjai_mul_assign(zjai_ctx* ctx, zjai_tensor* a, const zjai_tensor* b) { return eltwise(ctx, EL_MUL, a, b); }
extern "C" int32_t zjai_elu_gate(zjai_ctx* ctx, zjai_tensor* a, const zjai_tensor* b) { return eltwise(ctx, EL_ELU_GATE, a, b); }

extern "C" int32_t zjai_pixel_shuffle(zjai_ctx* ctx, const zjai_tensor* x, int32_t r, zjai_tensor** out) {
    if (!ctx || !x || !out) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        const Tensor& a = *x->t;
        need(r > 0 && a.c % (r * r) == 0, "pixel_shuffle: channels not divisible by r^2");
        const int co = a.c / (r * r);
        need(co % 4 == 0, "pixel_shuffle: output channels must be a multiple of 4");
        TensorP y = ctx->c.alloc(a.n, co, a.h * r, a.w * r, a.dtype);
        LaunchScope sc(ctx->c, kname("k_pixel_shuffle", a.dtype), 0.0, 2.0 * dtype_size(a.dtype) * a.c * a.h * a.w);
        ZJAI_HIP(launch_pixel_shuffle(a.v, y->v, a.dtype, a.n, co, a.h, a.w, r, ctx->c.stream));
        *out = new zjai_tensor{y};
    });
}

extern "C" int32_t zjai_layer_norm_channels(zjai_ctx* ctx, const zjai_tensor* x, const float* weight,
                                            const float* bias, zjai_tensor** out) {
    if (!ctx || !x || !weight || !bias || !out) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        const Tensor& a = *x->t;
        need(a.c % 4 == 0, "layer norm: channel count must be a multiple of 4");
        float* d = (float*)ctx->c.pool.alloc(sizeof(float) * 2 * a.c);
        std::shared_ptr<void> keep(d, [ctx](void* q) { ctx->c.pool.release(q); });
        ZJAI_HIP(hipMemcpyAsync(d, weight, sizeof(float) * a.c, hipMemcpyHostToDevice, ctx->c.stream));
        ZJAI_HIP(hipMemcpyAsync(d + a.c, bias, sizeof(float) * a.c, hipMemcpyHostToDevice, ctx->c.stream));
        TensorP y = ctx->c.alloc(a.n, a.c, a.h, a.w, a.dtype);
        {
            LaunchScope sc(ctx->c, kname("k_layer_norm", a.dtype), 0.0, 2.0 * dtype_size(a.dtype) * a.c * a.h * a.w);
            ZJAI_HIP(launch_layer_norm(a.v, y->v, a.dtype, a.n, a.c, a.h, a.w, d, d + a.c, ctx->c.stream));
        }
        ZJAI_HIP(hipStreamSynchronize(ctx->c.stream));
        *out = new zjai_tensor{y};
    });
}

extern "C" int32_t zjai_channel_attention(zjai_ctx* ctx, const zjai_tensor* qkv, int32_t heads,
                                          const float* temperature, zjai_tensor** out) {
    if (!ctx || !qkv || !temperature || !out) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        const Tensor& a = *qkv->t;
        need(heads > 0 && a.c % (3 * heads) == 0, "attention: channel / head counts");
        const int dim = a.c / 3, c = dim / heads;
        need(dim % 8 == 0, "attention: dim must be a multiple of 8");
        need(c >= 1 && c <= 32, "attention: at most 32 channels per head");
        if (!attention_gram_fits(a.dtype, dim)) throw Error(ZJAI_E_UNSUPPORTED, "attention: dim too large for the Gram kernel's LDS stage");
        // attn . v as a 1x1 conv over v with the block-diagonal attention matrix as its weight
        // (identity projection folded in).
        std::vector<float> eye((size_t)dim * dim, 0.0f);
        for (int i = 0; i < dim; ++i) eye[(size_t)i * dim + i] = 1.0f;
        LayerP L = make_conv(ctx->c, dim, dim, 1, 1, 1, 0, 0, 1, eye.data(), nullptr, nullptr, a.dtype, true);
        float* temp = (float*)ctx->c.pool.alloc(sizeof(float) * heads);
        std::shared_ptr<void> kt(temp, [ctx](void* q) { ctx->c.pool.release(q); });
        ZJAI_HIP(hipMemcpyAsync(temp, temperature, sizeof(float) * heads, hipMemcpyHostToDevice, ctx->c.stream));
        Epilogue e;
        std::shared_ptr<void> wfold = attention_fold(ctx->c, qkv->t, heads, temp, *L, &e.w_bstride);
        e.w_batch = wfold.get();
        TensorP y = conv_forward(ctx->c, *L, channel_view(qkv->t, 2 * dim, dim), e);
        ZJAI_HIP(hipStreamSynchronize(ctx->c.stream));
        *out = new zjai_tensor{y};
    });
}

extern "C" int32_t zjai_channel_attention_noalloc(zjai_ctx* ctx, const void* qkv, int32_t channels,
                                                  int32_t h, int32_t w, int32_t heads,
                                                  const float* temperature, int32_t precision,
                                                  void* out) {
    if (!ctx || !qkv || !temperature || !out) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        need(precision >= DT_F32 && precision <= DT_BF16, "precision");
        need(h > 0 && w > 0, "attention: empty map");
        need(heads > 0 && channels > 0 && channels % (3 * heads) == 0, "attention: channel / head counts");
        const int dim = channels / 3, c = dim / heads;
        need(dim % 8 == 0, "attention: dim must be a multiple of 8");
        need(c >= 1 && c <= 32, "attention: at most 32 channels per head");
        if (!attention_gram_fits(precision, dim)) throw Error(ZJAI_E_UNSUPPORTED, "attention: dim too large for the Gram kernel's LDS stage");
        need((((uintptr_t)qkv | (uintptr_t)out) & 15) == 0 && ((uintptr_t)temperature & 3) == 0,
             "attention: buffers not aligned (16 bytes; temperature 4)");
        // The dim x dim 1x1 projection (the identity) the attention is folded into, in the
        // packing make_conv gives it: [chunk][nblk][16][CK] of the storage type.
        const int es = dtype_size(precision), CK = 64 / es;
        const TileCfg cfg = conv_tile_cfg(dim, CK_1x1, precision);
        const int nblk = round_up(ceil_div(dim, 16), cfg.wc * cfg.cf), nchunks = ceil_div(dim, CK);
        const size_t w_bytes = (size_t)nchunks * nblk * 16 * CK * es;
        // Scratch layout: Gram partials [nchunk][heads][c*c + 2c] f32 | attn [dim][c] f32 | weight.
        const int nchunk = attention_gram_chunks(h, w);
        const size_t part_bytes = (size_t)nchunk * heads * (c * c + 2 * c) * 4;
        const size_t attn_off = round_up256(part_bytes), w_off = round_up256(attn_off + (size_t)dim * c * 4);
        if (w_off + w_bytes > ZJAI_NOALLOC_SCRATCH_BYTES)
            throw Error(ZJAI_E_LIMIT, "attention: the map needs more than the allocation-free scratch");
        unsigned char* base = scratch_of(ctx->c.device);
        if (!base) throw Error(ZJAI_E_DEVICE, "allocation-free scratch not set up for this device");
        float* partial = (float*)base;
        float* attn = (float*)(base + attn_off);
        void* wfold = base + w_off;
        Context& C = ctx->c;
        const View vq{const_cast<void*>(qkv), (long long)w * channels, (long long)h * w * channels, channels, 0};
        // Padded rows / columns of the folded weight must read zero, and the scratch keeps the
        // last call's contents.
        if (nblk * 16 != dim || nchunks * CK != dim) {
            LaunchScope sc(C, "k_zero_u32", 0.0, (double)w_bytes);
            ZJAI_HIP(launch_zero(wfold, w_bytes, C.stream));
        }
        const double n = (double)h * w, total = (double)heads * (c * c + 2 * c);
        {
            LaunchScope sc(C, attention_gram_name(vq, precision, dim, heads, w), 2.0 * total * n, es * 2.0 * dim * n + 4.0 * nchunk * total);
            ZJAI_HIP(launch_attention_gram(vq, precision, 1, dim, heads, h, w, partial, C.stream));
        }
        {
            LaunchScope sc(C, "k_attention_softmax", 0.0, 4.0 * nchunk * total);
            ZJAI_HIP(launch_attention_softmax(partial, 1, nchunk, dim, heads, temperature, attn, C.stream));
        }
        {
            LaunchScope sc(C, kname("k_attention_fold", precision), 2.0 * dim * dim * c, 4.0 * dim * c + (double)w_bytes);
            ZJAI_HIP(launch_attention_fold(nullptr, attn, 1, dim, heads, precision, nblk, wfold,
                                           (long long)(w_bytes / es), C.stream));
        }
        // attn . v: the folded weight as a 1x1 conv over the v channels (conv_forward's launch).
        ConvParams p{};
        p.x = View{const_cast<void*>(qkv), (long long)w * channels, (long long)h * w * channels, channels, 2 * dim};
        p.H = h;
        p.W = w;
        p.N = 1;
        p.OH = h;
        p.OW = w;
        p.y = View{out, (long long)w * dim, (long long)h * w * dim, dim, 0};
        p.w = wfold;
        p.w_bstride = (long long)(w_bytes / es);
        p.bias = nullptr;
        p.cin_g = dim;
        p.cout_g = dim;
        p.groups = 1;
        p.nchunks = nchunks;
        p.nblk_g = nblk;
        p.ntiles = nblk / (cfg.wc * cfg.cf);
        p.ps = 1;
        p.out_mode = OUT_NHWC;
        p.sv = p.sh = 1;
        LaunchScope sc(C, conv_kernel_name(CK_1x1, precision, cfg), 2.0 * n * dim * dim, es * 2.0 * n * dim + (double)w_bytes);
        ZJAI_HIP(launch_conv(CK_1x1, precision, cfg, p, C.stream));
    });
}

// ----------------------------------------------------------------------------------- nets
static std::map<std::string, Param> params_of(int32_t n_tensors, const char* const* names, const int32_t* ndims,
                                              const int32_t* dims, const float* const* data) {
    std::map<std::string, Param> P;
    const int32_t* d = dims;
    for (int i = 0; i < n_tensors; ++i) {
        need(names[i] != nullptr && ndims[i] >= 0 && ndims[i] <= 8, "tensor descriptor");
        Param p;
        p.shape.assign(d, d + ndims[i]);
        d += ndims[i];
        p.data = data[i];
        P[names[i]] = p;
    }
    return P;
}

extern "C" int32_t zjai_net_create(zjai_ctx* ctx, int32_t op, int32_t component, int32_t precision,
                                   int32_t n_tensors, const char* const* names, const int32_t* ndims,
                                   const int32_t* dims, const float* const* data, zjai_net** out) {
    if (!ctx || !out || n_tensors < 0 || (n_tensors && (!names || !ndims || !dims || !data)))
        return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        need(precision >= DT_F32 && precision <= DT_BF16, "precision");
        *out = new zjai_net{build_net(ctx->c, op, component, precision, params_of(n_tensors, names, ndims, dims, data))};
    });
}

extern "C" int32_t zjai_net_destroy(zjai_net* net) {
    delete net;
    return ZJAI_OK;
}

extern "C" int32_t zjai_net_out_size(const zjai_net* net, int32_t h, int32_t w, int32_t* oh, int32_t* ow) {
    if (!net || !oh || !ow || h <= 0 || w <= 0 || net->n->kind != NET_SYNTHESIS) return ZJAI_E_INVALID_ARGUMENT;
    if (net->n->comp == COMP_Y) primary_out_size(net->n->op, h, w, oh, ow);
    else secondary_out_size(net->n->op, h, w, oh, ow);
    return ZJAI_OK;
}

extern "C" int32_t zjai_net_device_bytes(const zjai_net* net, uint64_t* bytes) {
    if (!net || !bytes) return ZJAI_E_INVALID_ARGUMENT;
    *bytes = net->n->device_bytes();
    return ZJAI_OK;
}

static void run_to_host(zjai_ctx* ctx, const zjai_net* net, const TensorP& a, const TensorP& b, int h, int w,
                        float* out, size_t len) {
    const bool primary = net->n->comp == COMP_Y;
    int oh, ow;
    if (primary) primary_out_size(net->n->op, h, w, &oh, &ow);
    else secondary_out_size(net->n->op, h, w, &oh, &ow);
    const int planes = primary ? 1 : 2;
    const size_t n = (size_t)planes * oh * ow;
    need(out && len >= n, "output buffer too small");
    need(h > 0 && w > 0, "target size");
    float* dev = (float*)ctx->c.pool.alloc(n * 4);
    std::shared_ptr<void> keep(dev, [ctx](void* q) { ctx->c.pool.release(q); });
    PlaneOut po;
    po.plane = dev;
    po.row = ow;
    po.cstride = (long long)oh * ow;
    po.win_h[0] = oh;
    po.win_w[0] = ow;
    if (primary) primary_forward(ctx->c, *net->n, a, h, w, po);
    else secondary_forward(ctx->c, *net->n, a, b, h, w, po);
    ZJAI_HIP(hipMemcpyAsync(out, dev, n * 4, hipMemcpyDeviceToHost, ctx->c.stream));
    ZJAI_HIP(hipStreamSynchronize(ctx->c.stream));
}

extern "C" int32_t zjai_primary_forward(zjai_ctx* ctx, const zjai_net* net, const zjai_tensor* y_hat,
                                        int32_t h, int32_t w, float* out, size_t len) {
    if (!ctx || !net || !y_hat) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        need(net->n->kind == NET_SYNTHESIS && net->n->comp == COMP_Y, "not a primary net");
        need(y_hat->t->dtype == net->n->dtype, "latent precision differs from the net");
        run_to_host(ctx, net, y_hat->t, nullptr, h, w, out, len);
    });
}

extern "C" int32_t zjai_secondary_forward(zjai_ctx* ctx, const zjai_net* net, const zjai_tensor* y_luma,
                                          const zjai_tensor* y_chroma, int32_t h, int32_t w, float* out,
                                          size_t len) {
    if (!ctx || !net || !y_luma || !y_chroma) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        need(net->n->kind == NET_SYNTHESIS && net->n->comp == COMP_UV, "not a secondary net");
        run_to_host(ctx, net, y_luma->t, y_chroma->t, h, w, out, len);
    });
}

// ------------------------------------------------------------------------ tiling geometry
// synthesis_tiles / region_tiles / latent_extent (src/tools/tiles.rs:39-229) and the image
// region grid of independent regions (src/tools/regions.rs:47-150).
namespace {

struct Area {
    int x, y, w, h;
};

bool contains(const Area& r, int x, int y) { return r.x <= x && x < r.x + r.w && r.y <= y && y < r.y + r.h; }

int latent_extent(int pos, int len, int latent_len) {
    if (len % 16 && ceil_div(pos + len, 16) < latent_len)
        throw Error(ZJAI_E_INVALID_ARGUMENT, "unaligned synthesis tile inside the picture");
    return ceil_div(len, 16);
}

std::vector<std::pair<int, int>> axis_coords(int size, int n) {
    const int region = (ceil_div(size, 128) / n) * 128;
    std::vector<std::pair<int, int>> out;
    for (int i = 0; i < n; ++i) out.push_back({i * region, i + 1 < n ? (i + 1) * region : size});
    return out;
}

}  // namespace

extern "C" int32_t zjai_synthesis_tiles(int32_t height, int32_t width, int32_t latent_h, int32_t latent_w,
                                        int32_t tile_size, int32_t overlap, int32_t region_rows,
                                        int32_t region_cols, zjai_tile* tiles, int32_t cap, int32_t* n) {
    if (!n || height <= 0 || width <= 0 || latent_h <= 0 || latent_w <= 0 || cap < 0 || (cap && !tiles))
        return ZJAI_E_INVALID_ARGUMENT;
    return guard(nullptr, [&] {
        std::vector<zjai_tile> out;
        auto push = [&](Area img, Area lat, Area core, int ox, int oy) {
            out.push_back(zjai_tile{img.x, img.y, img.w, img.h, lat.x, lat.y, lat.w, lat.h, core.x, core.y,
                                    core.w, core.h, ox, oy});
        };
        if (tile_size <= 0) {
            Area img{0, 0, width, height};
            push(img, Area{0, 0, latent_w, latent_h}, img, 0, 0);
        } else {
            const int tile_h = std::min(tile_size, height), tile_w = std::min(tile_size, width);
            const int half = overlap / 2;
            if (region_rows > 0 && region_cols > 0) {
                std::vector<Area> regions;
                for (auto& vy : axis_coords(height, region_rows))
                    for (auto& vx : axis_coords(width, region_cols))
                        regions.push_back(Area{vx.first, vy.first, vx.second - vx.first, vy.second - vy.first});
                for (int ty = 0; ty < height; ty += tile_h)
                    for (int tx = 0; tx < width; tx += tile_w) {
                        int x = tx, y = ty, w = std::min(tile_w, width - tx), h = std::min(tile_h, height - ty);
                        const int x_end = x + w - 1, y_end = y + h - 1;
                        for (const Area& r : regions) {
                            if (!(contains(r, x, y) && contains(r, x_end, y_end))) continue;
                            if (y > r.y) {
                                if (y < half) throw Error(ZJAI_E_INVALID_ARGUMENT, "tile overlap");
                                y -= half;
                                h += half;
                            }
                            if (x > r.x) {
                                if (x < half) throw Error(ZJAI_E_INVALID_ARGUMENT, "tile overlap");
                                x -= half;
                                w += half;
                            }
                            if (y_end < r.y + r.h - 1) h += std::min(half, std::max(height - (y + h), 0));
                            if (x_end < r.x + r.w - 1) w += std::min(half, std::max(width - (x + w), 0));
                        }
                        if (x + w > width || y + h > height)
                            throw Error(ZJAI_E_INVALID_ARGUMENT, "synthesis tile outside the picture");
                        Area lat{x / 16, y / 16, latent_extent(x, w, latent_w), latent_extent(y, h, latent_h)};
                        if (lat.x + lat.w > latent_w || lat.y + lat.h > latent_h)
                            throw Error(ZJAI_E_INVALID_ARGUMENT, "synthesis tile outside the latent");
                        int cx = x, cy = y, cw = w, chh = h, left = 0, top = 0;
                        const int bx = x + w - 1, by = y + h - 1;
                        for (const Area& r : regions) {
                            if (!(contains(r, cx, cy) && contains(r, bx, by))) continue;
                            if (cy > r.y) {
                                top += half;
                                cy += half;
                                if (chh < half) throw Error(ZJAI_E_INVALID_ARGUMENT, "tile overlap");
                                chh -= half;
                            }
                            if (cx > r.x) {
                                left += half;
                                cx += half;
                                if (cw < half) throw Error(ZJAI_E_INVALID_ARGUMENT, "tile overlap");
                                cw -= half;
                            }
                            chh = std::min(chh, tile_h);
                            cw = std::min(cw, tile_w);
                        }
                        if (cw == 0 || chh == 0 || left + cw > w || top + chh > h)
                            throw Error(ZJAI_E_INVALID_ARGUMENT, "synthesis tile is all overlap");
                        push(Area{x, y, w, h}, lat, Area{cx, cy, cw, chh}, left, top);
                    }
            } else {
                if (tile_h <= overlap || tile_w <= overlap)
                    throw Error(ZJAI_E_INVALID_ARGUMENT, "synthesis tile not larger than its overlap");
                for (int y = 0; y < height - overlap; y += tile_h - overlap)
                    for (int x = 0; x < width - overlap; x += tile_w - overlap) {
                        Area img{x, y, std::min(tile_w, width - x), std::min(tile_h, height - y)};
                        Area lat{x / 16, y / 16, latent_extent(img.x, img.w, latent_w),
                                 latent_extent(img.y, img.h, latent_h)};
                        if (lat.x + lat.w > latent_w || lat.y + lat.h > latent_h)
                            throw Error(ZJAI_E_INVALID_ARGUMENT, "synthesis tile outside the latent");
                        const int left = img.x == 0 ? 0 : half, top = img.y == 0 ? 0 : half;
                        const int right = img.x + img.w >= width ? 0 : half;
                        const int bottom = img.y + img.h >= height ? 0 : half;
                        if (img.w <= left + right || img.h <= top + bottom)
                            throw Error(ZJAI_E_INVALID_ARGUMENT, "synthesis tile is all overlap");
                        push(img, lat, Area{img.x + left, img.y + top, img.w - left - right, img.h - top - bottom},
                             left, top);
                    }
            }
        }
        *n = (int32_t)out.size();
        if ((int)out.size() > cap) throw Error(ZJAI_E_LIMIT, "tile buffer too small");
        std::copy(out.begin(), out.end(), tiles);
    });
}

// ------------------------------------------------------------------- picture plan and memory
// A picture's tiles checked and grouped into batches: tiles of one image and latent window size
// share every layer shape and run as one batch of up to MAXB, in the order of their sizes; with
// lanes > 1 batch i runs on lane i % lanes. Host only.
struct PicturePlan {
    std::vector<std::vector<int>> batches;
    std::vector<zjai_tile> tiles;
    int op = 0, dtype = DT_F32, lh = 0, lw = 0, out_h = 0, out_w = 0, sv = 1, sh = 1, bit_depth = 0;
    bool uv = false;
};

static PicturePlan plan_picture(int op, int dtype, bool uv, int lh, int lw, int height, int width,
                                const zjai_tile* tiles, int n_tiles, int sv, int sh, int out_h, int out_w,
                                int bit_depth) {
    need(op >= OP_SOP && op <= OP_HOP, "operating point");
    need(dtype >= DT_F32 && dtype <= DT_BF16, "precision");
    need(tiles && n_tiles > 0, "no tiles");
    need(lh > 0 && lw > 0 && height > 0 && width > 0, "sizes");
    need(sv >= 1 && sv <= 2 && sh >= 1 && sh <= 2, "chroma subsampling");
    need(out_h > 0 && out_w > 0 && out_h <= height && out_w <= width, "displayed size");
    need(bit_depth == 0 || (bit_depth >= 8 && bit_depth <= 16), "bit depth");
    PicturePlan p;
    p.op = op; p.dtype = dtype; p.uv = uv; p.lh = lh; p.lw = lw; p.out_h = out_h; p.out_w = out_w;
    p.sv = sv; p.sh = sh; p.bit_depth = bit_depth;
    p.tiles.assign(tiles, tiles + n_tiles);
    for (const zjai_tile& t : p.tiles) {
        need(t.latent_x >= 0 && t.latent_y >= 0 && t.latent_w > 0 && t.latent_h > 0 &&
                 t.latent_x + t.latent_w <= lw && t.latent_y + t.latent_h <= lh,
             "tile latent window outside the latent");
        need(t.image_w > 0 && t.image_h > 0 && t.core_w > 0 && t.core_h > 0, "tile sizes");
        // latent_extent (src/tools/tiles.rs:22-24): a tile's latent window is ceil(len / 16).
        need(t.latent_h == ceil_div(t.image_h, 16) && t.latent_w == ceil_div(t.image_w, 16),
             "tile latent window is not ceil(image size / 16)");
        int oh, ow;
        primary_out_size(op, t.image_h, t.image_w, &oh, &ow);
        need(t.core_off_y >= 0 && t.core_off_x >= 0 && t.core_off_y + t.core_h <= oh &&
                 t.core_off_x + t.core_w <= ow,
             "synthesis tile smaller than its core");
        need(t.core_x >= 0 && t.core_y >= 0, "tile core position");
    }
    std::map<std::array<int, 4>, std::vector<int>> by_size;
    for (int i = 0; i < n_tiles; ++i) {
        const zjai_tile& t = p.tiles[i];
        by_size[{t.image_h, t.image_w, t.latent_h, t.latent_w}].push_back(i);
    }
    for (auto& kv : by_size)
        for (size_t i = 0; i < kv.second.size(); i += MAXB)
            p.batches.emplace_back(kv.second.begin() + i, kv.second.begin() + std::min(kv.second.size(), i + MAXB));
    return p;
}

// Device memory of one picture, the counterpart of the reference's `estimate_memory`
// (src/decoder/limits.rs:164-245), which sizes a decode from its header before anything runs as
// fixed buffers plus bytes per sample of the synthesis tiles.
//  * picture: the latents and output planes zjai_picture_create allocates (exact).
//  * live: the pool blocks in use at once (a model). A batch of N tiles of one latent window holds
//    at most KL x N x 256 x latent_h x latent_w bytes (16 x 16 samples per latent position: the
//    extent every layer's map scales with) and frees them all at its end; lanes run their batches
//    at the same time, so live = sum over lanes of the largest batch each runs.
//  * pool: the blocks the pools keep (a model). A pool reuses a cached block only for a request of
//    the same size up to 1.5x larger, so a lane keeps the blocks of every (tile shape, batch size)
//    it ran: sum over those of KP x N x 256 x latent_h x latent_w.
// KL and KP are measured (pool_peak and pool_cached after one 1024 x 1024 untiled picture on a
// released context; the same per-sample figures from 256 x 256 up), plus 8 %, and 256 KiB per
// term for the pool's size rounding on small tiles.
struct MemEstimate {
    uint64_t picture = 0, live = 0, pool = 0;
};

static MemEstimate estimate_picture(const PicturePlan& p, int lanes) {
    // Measured bytes per sample and batch item: [op][16-bit storage][with a chroma net].
    static const double KL[3][2][2] = {
        {{18.5, 18.5}, {9.2, 9.2}},        // SOP
        {{50.5, 50.5}, {25.2, 25.2}},      // BOP
        {{290.5, 290.5}, {145.2, 145.2}},  // HOP
    };
    static const double KP[3][2][2] = {
        {{29.0, 32.5}, {14.5, 16.2}},
        {{93.0, 110.5}, {46.5, 55.2}},
        {{517.0, 630.0}, {260.8, 318.7}},
    };
    const int s16 = p.dtype == DT_F32 ? 0 : 1, u = p.uv ? 1 : 0;
    const double kl = KL[p.op][s16][u] * 1.08, kp = KP[p.op][s16][u] * 1.08, slack = 256.0 * 1024.0;
    MemEstimate e;
    const uint64_t lat = (uint64_t)p.lh * p.lw, sb = p.bit_depth ? 2 : 4;
    e.picture = 4 * 160 * lat + sb * (uint64_t)p.out_h * p.out_w;
    if (p.uv) e.picture += 4 * 96 * lat + sb * 2 * (uint64_t)ceil_div(p.out_h, p.sv) * ceil_div(p.out_w, p.sh);
    const int nl = std::max(1, std::min<int>(lanes, (int)p.batches.size()));
    std::vector<std::set<std::array<int, 3>>> held(nl);
    for (size_t i = 0; i < p.batches.size(); ++i) {
        const zjai_tile& t = p.tiles[p.batches[i][0]];
        held[i % nl].insert({t.latent_h, t.latent_w, (int)p.batches[i].size()});
    }
    double live = 0.0, pool = 0.0;
    for (const auto& lane : held) {
        double top = 0.0;
        for (const auto& s : lane) {
            const double samples = (double)s[2] * 256.0 * s[0] * s[1];
            top = std::max(top, kl * samples);
            pool += kp * samples + slack;
        }
        live += top + slack;
    }
    e.live = (uint64_t)std::ceil(live);
    e.pool = (uint64_t)std::ceil(pool);
    return e;
}

// Admission: with a memory limit set on the context, a picture whose nets, buffers and modelled
// live pool blocks exceed it is refused before anything is allocated (the reference checks its
// estimate's live bytes against `max_memory_bytes` the same way, src/decoder/limits.rs:106-111).
static void admit(const Context& c, const PicturePlan& p, int lanes, const Net& net_y, const Net* net_uv) {
    if (!c.mem_limit) return;
    const MemEstimate e = estimate_picture(p, lanes);
    const uint64_t total = e.picture + e.live + net_y.device_bytes() + (net_uv ? net_uv->device_bytes() : 0);
    if (total > c.mem_limit)
        throw Error(ZJAI_E_LIMIT, "estimated device memory of the picture (" + std::to_string(total) +
                                      " bytes) exceeds the context's limit (" + std::to_string(c.mem_limit) +
                                      " bytes)");
}

extern "C" int32_t zjai_picture_estimate_memory(int32_t op, int32_t precision, int32_t with_uv, int32_t lh,
                                                int32_t lw, int32_t height, int32_t width,
                                                const zjai_tile* tiles, int32_t n_tiles, int32_t sv,
                                                int32_t sh, int32_t out_h, int32_t out_w, int32_t bit_depth,
                                                int32_t lanes, zjai_memory_estimate* out) {
    if (!out || !tiles || n_tiles <= 0 || lanes < 1 || lanes > MAXB || (with_uv != 0 && with_uv != 1))
        return ZJAI_E_INVALID_ARGUMENT;
    return guard(nullptr, [&] {
        const PicturePlan p = plan_picture(op, precision, with_uv != 0, lh, lw, height, width, tiles, n_tiles,
                                           sv, sh, out_h, out_w, bit_depth);
        const MemEstimate e = estimate_picture(p, lanes);
        out->picture_bytes = e.picture;
        out->live_bytes = e.live;
        out->pool_bytes = e.pool;
    });
}

extern "C" int32_t zjai_ctx_set_memory_limit(zjai_ctx* ctx, uint64_t bytes) {
    if (!ctx) return ZJAI_E_INVALID_ARGUMENT;
    ctx->c.mem_limit = bytes;
    return ZJAI_OK;
}

// --------------------------------------------------------------------------------- picture
struct zjai_picture {
    NetP net_y, net_uv;
    int lh = 0, lw = 0, height = 0, width = 0, sv = 1, sh = 1, out_h = 0, out_w = 0, bit_depth = 0;
    std::vector<zjai_tile> tiles;
    std::vector<std::vector<int>> batches;  // tile indices of equal image size, at most MAXB each
    int lanes = 1;            // tile batches run on this many concurrent streams
    std::vector<hipEvent_t> lane_ev;  // join events, one per lane
    float* y_hat = nullptr;   // device planar [160][lh][lw]
    float* uv_hat = nullptr;  // device planar [96][lh][lw]
    void* out_y = nullptr;    // device planes
    void* out_uv = nullptr;   // [2][ch][cw]
    uint16_t* out_rgb = nullptr;  // [out_h][out_w][3] (zjai_picture_download_rgb)
    float* out_rgbf = nullptr;    // [3][out_h][out_w]
    bool uploaded = false;
    // Replay (zjai_picture_set_replay): the run's launch sequence captured once as a HIP graph,
    // the pool blocks its launches address, its launch count and the lane count it was captured
    // with; fork is the event the lanes wait on inside the capture.
    bool replay = false;
    hipGraphExec_t gexec = nullptr;
    std::vector<void*> gbufs;
    long long glaunches = 0;
    int glanes = 0;
    hipEvent_t fork = nullptr;
    void drop_graph() {
        if (gexec) (void)hipGraphExecDestroy(gexec);
        gexec = nullptr;
        for (void* q : gbufs) (void)hipFree(q);
        gbufs.clear();
        glanes = 0;
    }
    ~zjai_picture() {
        drop_graph();
        if (fork) (void)hipEventDestroy(fork);
        for (hipEvent_t e : lane_ev) (void)hipEventDestroy(e);
        if (y_hat) (void)hipFree(y_hat);
        if (uv_hat) (void)hipFree(uv_hat);
        if (out_y) (void)hipFree(out_y);
        if (out_uv) (void)hipFree(out_uv);
        if (out_rgb) (void)hipFree(out_rgb);
        if (out_rgbf) (void)hipFree(out_rgbf);
    }
    size_t sample_bytes() const { return bit_depth ? 2 : 4; }
    int ch() const { return ceil_div(out_h, sv); }
    int cw() const { return ceil_div(out_w, sh); }
};

extern "C" int32_t zjai_picture_create(zjai_ctx* ctx, const zjai_net* net_y, const zjai_net* net_uv,
                                       int32_t lh, int32_t lw, int32_t height, int32_t width,
                                       const zjai_tile* tiles, int32_t n_tiles, int32_t sv, int32_t sh,
                                       int32_t out_h, int32_t out_w, int32_t bit_depth, zjai_picture** out) {
    if (!ctx || !net_y || !out || !tiles || n_tiles <= 0) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        need(net_y->n->kind == NET_SYNTHESIS && net_y->n->comp == COMP_Y, "net_y is not a primary net");
        need(!net_uv || (net_uv->n->kind == NET_SYNTHESIS && net_uv->n->comp == COMP_UV &&
                         net_uv->n->op == net_y->n->op),
             "net_uv mismatch");
        need(!net_uv || net_uv->n->dtype == net_y->n->dtype, "nets differ in precision");
        PicturePlan plan = plan_picture(net_y->n->op, net_y->n->dtype, net_uv != nullptr, lh, lw, height, width,
                                        tiles, n_tiles, sv, sh, out_h, out_w, bit_depth);
        admit(ctx->c, plan, 1, *net_y->n, net_uv ? net_uv->n.get() : nullptr);
        auto* p = new zjai_picture();
        std::unique_ptr<zjai_picture> own(p);
        p->net_y = net_y->n;
        if (net_uv) p->net_uv = net_uv->n;
        p->lh = lh; p->lw = lw; p->height = height; p->width = width; p->sv = sv; p->sh = sh;
        p->out_h = out_h; p->out_w = out_w; p->bit_depth = bit_depth;
        p->tiles.assign(tiles, tiles + n_tiles);
        p->batches = std::move(plan.batches);
        ZJAI_HIP(hipMalloc(&p->y_hat, sizeof(float) * 160 * (size_t)lh * lw));
        if (p->net_uv) ZJAI_HIP(hipMalloc(&p->uv_hat, sizeof(float) * 96 * (size_t)lh * lw));
        ZJAI_HIP(hipMalloc(&p->out_y, p->sample_bytes() * (size_t)out_h * out_w));
        ZJAI_HIP(hipMemset(p->out_y, 0, p->sample_bytes() * (size_t)out_h * out_w));
        if (p->net_uv) {
            ZJAI_HIP(hipMalloc(&p->out_uv, p->sample_bytes() * 2 * (size_t)p->ch() * p->cw()));
            ZJAI_HIP(hipMemset(p->out_uv, 0, p->sample_bytes() * 2 * (size_t)p->ch() * p->cw()));
        }
        *out = own.release();
    });
}

extern "C" int32_t zjai_picture_destroy(zjai_picture* pic) {
    delete pic;
    return ZJAI_OK;
}

extern "C" int32_t zjai_picture_upload(zjai_ctx* ctx, zjai_picture* pic, const float* y_hat, const float* uv_hat) {
    if (!ctx || !pic || !y_hat) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        need(!pic->net_uv || uv_hat, "chroma latent missing");
        ZJAI_HIP(hipMemcpyAsync(pic->y_hat, y_hat, sizeof(float) * 160 * (size_t)pic->lh * pic->lw,
                                hipMemcpyHostToDevice, ctx->c.stream));
        if (pic->net_uv)
            ZJAI_HIP(hipMemcpyAsync(pic->uv_hat, uv_hat, sizeof(float) * 96 * (size_t)pic->lh * pic->lw,
                                    hipMemcpyHostToDevice, ctx->c.stream));
        ZJAI_HIP(hipStreamSynchronize(ctx->c.stream));
        pic->uploaded = true;
    });
}

// Issues every tile batch of the picture: batch i on lane i % nl (nl > 1: the lanes first wait
// for `fork` on the root stream, and the root stream waits for every lane at the end).
static void issue_picture(Context& root, zjai_picture* pic, int nl, hipEvent_t fork) {
    const int dt = pic->net_y->dtype;
    if (nl > 1) {
        for (int i = 0; i < nl; ++i) ZJAI_HIP(hipStreamWaitEvent(root.lane(i).stream, fork, 0));
    }
    for (size_t bidx = 0; bidx < pic->batches.size(); ++bidx) {
        const std::vector<int>& group = pic->batches[bidx];
        Context& c = nl > 1 ? root.lane((int)bidx % nl) : root;
        c.check_stop();
        const zjai_tile& t0 = pic->tiles[group[0]];
        const int N = (int)group.size();
        Windows win{};
        PlaneOut py;
        py.plane = pic->out_y;
        py.row = pic->out_w;
        py.bit_depth = pic->bit_depth;
        for (int b = 0; b < N; ++b) {
            const zjai_tile& t = pic->tiles[group[b]];
            win.x0[b] = t.latent_x;
            win.y0[b] = t.latent_y;
            // synthesize_luma_into (src/decoder/reconstruct.rs:379-411): core rows/cols that
            // fall inside the displayed picture.
            py.win_y0[b] = t.core_off_y;
            py.win_x0[b] = t.core_off_x;
            py.win_h[b] = std::min(t.core_h, std::max(pic->out_h - t.core_y, 0));
            py.win_w[b] = std::min(t.core_w, std::max(pic->out_w - t.core_x, 0));
            py.dst_y0[b] = t.core_y;
            py.dst_x0[b] = t.core_x;
        }
        // With a chroma net both latents go into one 256-channel block (luma channels 0..159,
        // chroma 160..255): the chroma net's input concatenation is then that block as it stands.
        TensorP cat = pic->net_uv ? c.alloc(N, 256, t0.latent_h, t0.latent_w, dt) : nullptr;
        TensorP by = cat ? channel_view(cat, 0, 160) : c.alloc(N, 160, t0.latent_h, t0.latent_w, dt);
        {
            LaunchScope sc(c, kname("k_planar_to_nhwc", dt), 0.0, (4.0 + dtype_size(dt)) * N * 160 * t0.latent_h * t0.latent_w);
            ZJAI_HIP(launch_planar_to_nhwc(pic->y_hat, 160, pic->lh, pic->lw, win, N, t0.latent_h, t0.latent_w,
                                           by->v, dt, c.stream));
        }
        primary_forward(c, *pic->net_y, by, t0.image_h, t0.image_w, py);
        if (pic->net_uv) {
            TensorP buv = channel_view(cat, 160, 96);
            {
                LaunchScope sc(c, kname("k_planar_to_nhwc", dt), 0.0, (4.0 + dtype_size(dt)) * N * 96 * t0.latent_h * t0.latent_w);
                ZJAI_HIP(launch_planar_to_nhwc(pic->uv_hat, 96, pic->lh, pic->lw, win, N, t0.latent_h,
                                               t0.latent_w, buv->v, dt, c.stream));
            }
            // synthesize_chroma_into (src/decoder/reconstruct.rs:416-464)
            PlaneOut pu = py;
            pu.plane = pic->out_uv;
            pu.row = pic->cw();
            pu.cstride = (long long)pic->ch() * pic->cw();
            pu.sv = pic->sv;
            pu.sh = pic->sh;
            secondary_forward(c, *pic->net_uv, by, buv, t0.image_h, t0.image_w, pu);
        }
    }
    if (nl > 1) {
        for (int i = 0; i < nl; ++i) {
            ZJAI_HIP(hipEventRecord(pic->lane_ev[i], root.lane(i).stream));
            ZJAI_HIP(hipStreamWaitEvent(root.stream, pic->lane_ev[i], 0));
        }
    }
}

// Replay mode: captures issue_picture's launches on the root stream (and, through the fork
// event, on every lane) as one HIP graph instead of running them. Nothing executes during the
// capture, so the pools hand out and take back blocks exactly as in an eager run; afterwards the
// blocks the graph addresses leave the pools (pic->gbufs) so that no later allocation can take
// one while a replay writes it. Captures no memset or copy: only kernels and the fork / join
// event dependencies.
static void capture_picture(Context& root, zjai_picture* pic, int nl) {
    pic->drop_graph();
    need(!root.profiling, "replay: per-launch profiling is on (profile eager runs)");
    if (!pic->fork) ZJAI_HIP(hipEventCreateWithFlags(&pic->fork, hipEventDisableTiming));
    std::vector<Context*> ctxs{&root};
    for (int i = 0; i < nl && nl > 1; ++i) ctxs.push_back(&root.lane(i));
    std::vector<size_t> held;
    for (Context* c : ctxs) {
        range_slots_init(*c);
        held.push_back(c->pool.in_use());
    }
    const long long l0 = root.launches;
    ZJAI_HIP(hipStreamBeginCapture(root.stream, hipStreamCaptureModeRelaxed));
    hipGraph_t g = nullptr;
    try {
        ZJAI_HIP(hipEventRecord(pic->fork, root.stream));
        issue_picture(root, pic, nl, pic->fork);
    } catch (...) {
        // Join every lane back to the root stream so that the capture ends cleanly, then drop it.
        for (int i = 0; i < nl && nl > 1; ++i) {
            (void)hipEventRecord(pic->lane_ev[i], root.lane(i).stream);
            (void)hipStreamWaitEvent(root.stream, pic->lane_ev[i], 0);
        }
        if (hipStreamEndCapture(root.stream, &g) == hipSuccess && g) (void)hipGraphDestroy(g);
        root.launches = l0;
        throw;
    }
    ZJAI_HIP(hipStreamEndCapture(root.stream, &g));
    const hipError_t e = hipGraphInstantiate(&pic->gexec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    ZJAI_HIP(e);
    pic->glaunches = root.launches - l0;
    root.launches = l0;
    pic->glanes = nl;
    for (size_t i = 0; i < ctxs.size(); ++i) {
        if (ctxs[i]->pool.in_use() != held[i]) {
            pic->drop_graph();
            throw Error(ZJAI_E_DEVICE, "replay: a buffer of the captured run is still held");
        }
        ctxs[i]->pool.surrender(pic->gbufs);
    }
}

extern "C" int32_t zjai_picture_run(zjai_ctx* ctx, zjai_picture* pic) {
    if (!ctx || !pic) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        need(pic->uploaded, "latents not uploaded");
        Context& root = ctx->c;
        // Tiles of one image size share every layer shape: run them as one batch of up to MAXB
        // (each launch then covers all of them). Batches are independent (disjoint core
        // rectangles of the output planes, read-only latents), so with lanes > 1 batch i runs
        // on lane i % lanes, concurrently with the others; the root stream waits for all lanes.
        const int nl = std::min<int>(pic->lanes, (int)pic->batches.size());
        while ((int)pic->lane_ev.size() < nl) {
            hipEvent_t e;
            ZJAI_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
            pic->lane_ev.push_back(e);
        }
        if (pic->replay) {
            if (!pic->gexec || pic->glanes != nl) capture_picture(root, pic, nl);
            root.check_stop();
            ZJAI_HIP(hipEventRecord(root.ev0, root.stream));
            ZJAI_HIP(hipGraphLaunch(pic->gexec, root.stream));
            root.launches += pic->glaunches;
            ZJAI_HIP(hipEventRecord(root.ev1, root.stream));
            ZJAI_HIP(hipEventSynchronize(root.ev1));
            ZJAI_HIP(hipEventElapsedTime(&root.last_ms, root.ev0, root.ev1));
            return;
        }
        ZJAI_HIP(hipEventRecord(root.ev0, root.stream));
        // A failure or cancellation part way through leaves the other lanes' batches queued:
        // drain every stream before reporting it, so the picture and the context are idle and
        // reusable when the call returns.
        struct Drain {
            Context& root;
            int nl;
            bool armed = true;
            ~Drain() {
                if (!armed) return;
                for (int i = 0; i < nl && nl > 1; ++i) (void)hipStreamSynchronize(root.lane(i).stream);
                (void)hipStreamSynchronize(root.stream);
            }
        } drain{root, nl};
        issue_picture(root, pic, nl, root.ev0);
        drain.armed = false;
        ZJAI_HIP(hipEventRecord(root.ev1, root.stream));
        ZJAI_HIP(hipEventSynchronize(root.ev1));
        ZJAI_HIP(hipEventElapsedTime(&root.last_ms, root.ev0, root.ev1));
    });
}

extern "C" int32_t zjai_picture_set_replay(zjai_ctx* ctx, zjai_picture* pic, int32_t on) {
    if (!ctx || !pic || (on != 0 && on != 1)) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        pic->replay = on != 0;
        if (!pic->replay) pic->drop_graph();
    });
}

extern "C" int32_t zjai_picture_set_lanes(zjai_ctx* ctx, zjai_picture* pic, int32_t lanes) {
    if (!ctx || !pic || lanes < 1 || lanes > MAXB) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        if (ctx->c.mem_limit) {
            PicturePlan plan;
            plan.op = pic->net_y->op; plan.dtype = pic->net_y->dtype; plan.uv = (bool)pic->net_uv;
            plan.lh = pic->lh; plan.lw = pic->lw; plan.out_h = pic->out_h; plan.out_w = pic->out_w;
            plan.sv = pic->sv; plan.sh = pic->sh; plan.bit_depth = pic->bit_depth;
            plan.tiles = pic->tiles;
            plan.batches = pic->batches;
            admit(ctx->c, plan, lanes, *pic->net_y, pic->net_uv.get());
        }
        pic->lanes = lanes;
    });
}

extern "C" int32_t zjai_picture_download(zjai_ctx* ctx, zjai_picture* pic, void* y, void* u, void* v) {
    if (!ctx || !pic || !y) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        const size_t sb = pic->sample_bytes();
        ZJAI_HIP(hipMemcpyAsync(y, pic->out_y, sb * (size_t)pic->out_h * pic->out_w, hipMemcpyDeviceToHost,
                                ctx->c.stream));
        if (pic->net_uv) {
            need(u && v, "chroma outputs missing");
            const size_t n = (size_t)pic->ch() * pic->cw();
            ZJAI_HIP(hipMemcpyAsync(u, pic->out_uv, sb * n, hipMemcpyDeviceToHost, ctx->c.stream));
            ZJAI_HIP(hipMemcpyAsync(v, (char*)pic->out_uv + sb * n, sb * n, hipMemcpyDeviceToHost, ctx->c.stream));
        }
        ZJAI_HIP(hipStreamSynchronize(ctx->c.stream));
    });
}

extern "C" int32_t zjai_host_alloc(zjai_ctx* ctx, size_t bytes, void** out) {
    if (!ctx || !out || bytes == 0) return ZJAI_E_INVALID_ARGUMENT;
    *out = nullptr;
    return guard(ctx, [&] {
        void* p = nullptr;
        ZJAI_HIP(hipHostMalloc(&p, bytes, hipHostMallocDefault));
        *out = p;
    });
}

extern "C" int32_t zjai_host_free(zjai_ctx* ctx, void* p) {
    if (!p) return ZJAI_OK;
    return guard(ctx, [&] { ZJAI_HIP(hipHostFree(p)); });
}

// ------------------------------------------------------------------------- output stage
extern "C" int32_t zjai_resize(zjai_ctx* ctx, int32_t mode, const float* src, int32_t c, int32_t h,
                               int32_t w, int32_t out_h, int32_t out_w, float* dst) {
    if (!ctx || !src || !dst) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        need(mode == ZJAI_RESIZE_BICUBIC || mode == ZJAI_RESIZE_BILINEAR, "resize: unknown mode");
        need(c > 0 && h > 0 && w > 0 && out_h > 0 && out_w > 0, "resize: empty dimension");
        const size_t n_in = (size_t)c * h * w, n_out = (size_t)c * out_h * out_w;
        Context& cx = ctx->c;
        // Flat f32 scratch from the context's pool: [1][1][n / 8][8] tensors.
        TensorP a = cx.alloc(1, 8, 1, (int)((n_in + 7) / 8), DT_F32);
        TensorP b = cx.alloc(1, 8, 1, (int)((n_out + 7) / 8), DT_F32);
        ZJAI_HIP(hipMemcpyAsync(a->v.p, src, n_in * 4, hipMemcpyHostToDevice, cx.stream));
        {
            LaunchScope sc(cx, mode == ZJAI_RESIZE_BICUBIC ? "k_resize_bicubic" : "k_resize_bilinear",
                           0.0, 4.0 * (double)(n_in + n_out));
            ZJAI_HIP(launch_resize(mode, (const float*)a->v.p, c, h, w, (float*)b->v.p, out_h, out_w, cx.stream));
        }
        ZJAI_HIP(hipMemcpyAsync(dst, b->v.p, n_out * 4, hipMemcpyDeviceToHost, cx.stream));
        ZJAI_HIP(hipStreamSynchronize(cx.stream));
    });
}

extern "C" int32_t zjai_picture_download_rgb(zjai_ctx* ctx, zjai_picture* pic, int32_t bit_depth,
                                             uint16_t* rgb, float* rgb_planes) {
    if (!ctx || !pic || !rgb) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        need(bit_depth == 8 || bit_depth == 10, "output bit depth must be 8 or 10");
        need(pic->bit_depth == 0, "RGB output needs a picture with float planes (bit_depth 0)");
        need(pic->net_uv != nullptr, "RGB output needs the chroma planes");
        need(pic->uploaded, "picture latents have not been uploaded");
        Context& cx = ctx->c;
        const size_t n = (size_t)pic->out_h * pic->out_w;
        if (!pic->out_rgb) ZJAI_HIP(hipMalloc((void**)&pic->out_rgb, n * 3 * sizeof(uint16_t)));
        if (rgb_planes && !pic->out_rgbf) ZJAI_HIP(hipMalloc((void**)&pic->out_rgbf, n * 3 * sizeof(float)));
        const int ch = pic->ch(), cw = pic->cw();
        const float* u = (const float*)pic->out_uv;
        const float* v = u + (size_t)ch * cw;
        {
            LaunchScope sc(cx, "k_picture_rgb", 0.0,
                           (double)n * (4.0 + 6.0 + (rgb_planes ? 12.0 : 0.0)) + 8.0 * (double)ch * cw);
            ZJAI_HIP(launch_picture_rgb((const float*)pic->out_y, pic->out_h, pic->out_w, u, v, ch, cw, bit_depth,
                                        pic->out_rgb, rgb_planes ? pic->out_rgbf : nullptr, cx.stream));
        }
        ZJAI_HIP(hipMemcpyAsync(rgb, pic->out_rgb, n * 3 * sizeof(uint16_t), hipMemcpyDeviceToHost, cx.stream));
        if (rgb_planes)
            ZJAI_HIP(hipMemcpyAsync(rgb_planes, pic->out_rgbf, n * 3 * sizeof(float), hipMemcpyDeviceToHost, cx.stream));
        ZJAI_HIP(hipStreamSynchronize(cx.stream));
    });
}

// ------------------------------------------------------------------ latent reconstruction
static RegionParams region_params(const zjai_regions* r) {
    RegionParams p;
    if (!r) return p;
    need(r->num_ver >= 1 && r->num_hor >= 1, "region counts must be positive");
    need(r->hyper_decoder_overlap >= 0 && r->mcm_overlap >= 0, "negative region overlap");
    p.partitioned = true;
    p.independent = r->independent != 0;
    p.num_ver = r->num_ver;
    p.num_hor = r->num_hor;
    p.hyper_decoder_overlap = r->hyper_decoder_overlap;
    p.mcm_overlap = r->mcm_overlap;
    return p;
}

extern "C" int32_t zjai_region_grid(int32_t height, int32_t width, int32_t component, const zjai_regions* regions,
                                    int32_t plane, zjai_area* core, zjai_area* extended, int32_t cap, int32_t* n) {
    if (!n || cap < 0 || (cap > 0 && (!core || !extended))) return ZJAI_E_INVALID_ARGUMENT;
    return guard(nullptr, [&] {
        need(component == 0 || component == 1, "component");
        const RegionGrid g = region_grid(height, width, component, region_params(regions), plane);
        *n = (int32_t)g.core.size();
        if (*n > cap) throw Error(ZJAI_E_LIMIT, "zjai_region_grid: capacity too small");
        for (int i = 0; i < *n; ++i) {
            core[i] = zjai_area{g.core[i].x, g.core[i].y, g.core[i].w, g.core[i].h};
            extended[i] = zjai_area{g.extended[i].x, g.extended[i].y, g.extended[i].w, g.extended[i].h};
        }
    });
}

extern "C" int32_t zjai_latent_model_create(zjai_ctx* ctx, int32_t component, int32_t precision, int32_t n_tensors,
                                            const char* const* names, const int32_t* ndims, const int32_t* dims,
                                            const float* const* data, zjai_net** out) {
    if (!ctx || !out || n_tensors < 0 || (n_tensors && (!names || !ndims || !dims || !data)))
        return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        need(precision >= DT_F32 && precision <= DT_BF16, "precision");
        *out = new zjai_net{build_latent_net(ctx->c, component, precision, params_of(n_tensors, names, ndims, dims, data))};
    });
}

extern "C" int32_t zjai_latent_model_info(const zjai_net* net, int32_t* channels, int32_t* has_context) {
    if (!net || !channels || !has_context || net->n->kind != NET_LATENT) return ZJAI_E_INVALID_ARGUMENT;
    *channels = net->n->chs;
    *has_context = net->n->context ? 1 : 0;
    return ZJAI_OK;
}

extern "C" int32_t zjai_hyper_decoder_forward(zjai_ctx* ctx, const zjai_net* net, const int8_t* z_hat, int32_t c,
                                              int32_t zh, int32_t zw, int32_t out_h, int32_t out_w, float* psi,
                                              size_t len) {
    if (!ctx || !net || !z_hat || !psi) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        const Net& m = *net->n;
        need(m.kind == NET_LATENT, "not a latent model");
        need(c == m.chs && zh > 0 && zw > 0, "z_hat shape");
        need(out_h > 0 && out_w > 0 && out_h <= 2 * zh && out_w <= 2 * zw, "psi size");
        need(len >= (size_t)4 * c * out_h * out_w, "output buffer too small");
        Context& cx = ctx->c;
        const size_t zn = (size_t)c * zh * zw;
        void* zdev = cx.pool.alloc(zn);
        std::shared_ptr<void> keep(zdev, [&cx](void* q) { cx.pool.release(q); });
        ZJAI_HIP(hipMemcpyAsync(zdev, z_hat, zn, hipMemcpyHostToDevice, cx.stream));
        TensorP z = cx.alloc(1, c, zh, zw, m.dtype);
        {
            LaunchScope sc(cx, kname("k_i8_planar_to_nhwc", m.dtype), 0.0, (1.0 + dtype_size(m.dtype)) * zn);
            ZJAI_HIP(launch_i8_planar_to_nhwc((const int8_t*)zdev, c, zh, zw, Windows{}, 1, zh, zw, z->v, m.dtype,
                                              cx.stream));
        }
        TensorP t = hyper_decoder_forward(cx, m, z, out_h, out_w);
        const size_t pn = (size_t)4 * c * out_h * out_w;
        float* dev = (float*)cx.pool.alloc(pn * 4);
        std::shared_ptr<void> keep2(dev, [&cx](void* q) { cx.pool.release(q); });
        {
            LaunchScope sc(cx, kname("k_nhwc_to_planar", m.dtype), 0.0, (4.0 + dtype_size(m.dtype)) * pn);
            ZJAI_HIP(launch_nhwc_to_planar(t->v, m.dtype, 1, 4 * c, out_h, out_w, dev, cx.stream));
        }
        ZJAI_HIP(hipMemcpyAsync(psi, dev, pn * 4, hipMemcpyDeviceToHost, cx.stream));
        ZJAI_HIP(hipStreamSynchronize(cx.stream));
    });
}

extern "C" int32_t zjai_context_decompress(zjai_ctx* ctx, const zjai_net* net, const float* residual, int32_t c,
                                           int32_t h, int32_t w, const float* psi, int32_t psi_h, int32_t psi_w,
                                           float* y_hat, size_t len) {
    if (!ctx || !net || !residual || !psi || !y_hat) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        const Net& m = *net->n;
        need(m.kind == NET_LATENT, "not a latent model");
        need(c == m.chs && h > 0 && w > 0 && psi_h > 0 && psi_w > 0, "residual / psi shape");
        need(len >= (size_t)c * h * w, "output buffer too small");
        Context& cx = ctx->c;
        const size_t rn = (size_t)c * h * w;
        TensorP ps = planar_upload(cx, psi, 4 * c, psi_h, psi_w, m.dtype);
        float* rdev = (float*)cx.pool.alloc(rn * 4);
        std::shared_ptr<void> keep(rdev, [&cx](void* q) { cx.pool.release(q); });
        float* ydev = (float*)cx.pool.alloc(rn * 4);
        std::shared_ptr<void> keep2(ydev, [&cx](void* q) { cx.pool.release(q); });
        ZJAI_HIP(hipMemcpyAsync(rdev, residual, rn * 4, hipMemcpyHostToDevice, cx.stream));
        latent_decompress(cx, m, rdev, w, (long long)h * w, Windows{}, h, w, ps, ydev);
        ZJAI_HIP(hipMemcpyAsync(y_hat, ydev, rn * 4, hipMemcpyDeviceToHost, cx.stream));
        ZJAI_HIP(hipStreamSynchronize(cx.stream));
    });
}

extern "C" int32_t zjai_reconstruct_latent(zjai_ctx* ctx, const zjai_net* net, int32_t height, int32_t width,
                                           const zjai_regions* regions, const int8_t* z_hat, int32_t zh, int32_t zw,
                                           const float* residual, int32_t h, int32_t w, float* psi, float* y_hat) {
    if (!ctx || !net || !z_hat || !residual || !psi || !y_hat) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        need(net->n->kind == NET_LATENT, "not a latent model");
        reconstruct_latent(ctx->c, *net->n, height, width, region_params(regions), z_hat, zh, zw, residual, h, w, psi,
                           y_hat);
    });
}

// ------------------------------------------------------------------------- weight readers
struct zjai_checkpoint {
    std::unique_ptr<Checkpoint> ck;
};
struct zjai_bundle {
    Bundle b;
};

namespace {

// A NUL-terminated copy of `s` into buf (ZJAI_E_LIMIT when it does not fit).
void copy_name(const std::string& s, char* buf, size_t cap) {
    need(buf != nullptr, "null name buffer");
    if (s.size() + 1 > cap) throw Error(ZJAI_E_LIMIT, "name buffer too small");
    std::memcpy(buf, s.data(), s.size());
    buf[s.size()] = 0;
}

const CkTensor& tensor_of(const zjai_checkpoint* ck, const char* name) {
    need(ck != nullptr && name != nullptr, "null checkpoint or name");
    const CkTensor* t = ck->ck->find(name);
    if (!t) throw Error(ZJAI_E_MODEL, std::string("tensor `") + name + "` not found");
    return *t;
}

// Every f32 / f16 tensor of a checkpoint as named f32 parameters; `hold` owns the data.
std::map<std::string, Param> checkpoint_params(const Checkpoint& ck, std::vector<std::vector<float>>& hold) {
    std::map<std::string, Param> P;
    hold.reserve(ck.tensors().size() + ck.lists().size());
    for (const CkTensor& t : ck.tensors()) {
        if (t.dtype != CK_F32 && t.dtype != CK_F16) continue;
        if (P.count(t.name)) continue;  // the first of duplicate names, as a by-name lookup finds
        Param p;
        for (uint64_t d : t.shape) {
            if (d > (uint64_t)INT32_MAX) throw Error(ZJAI_E_MODEL, "tensor `" + t.name + "`: dimension too large");
            p.shape.push_back((int)d);
        }
        hold.push_back(ck.f32(t));
        p.data = hold.back().data();
        P[t.name] = p;
    }
    // numeric lists (`clip_thres.E1B.MinList`, ...) as 1-D f32 parameters (`x as f32`)
    for (const auto& l : ck.lists()) {
        if (P.count(l.first)) continue;
        Param p;
        p.shape = {(int)l.second.size()};
        hold.emplace_back(l.second.begin(), l.second.end());
        p.data = hold.back().data();
        P[l.first] = p;
    }
    return P;
}

}  // namespace

extern "C" int32_t zjai_checkpoint_parse(const void* data, size_t len, zjai_checkpoint** out) {
    if (!out || (!data && len)) return ZJAI_E_INVALID_ARGUMENT;
    *out = nullptr;
    return guard(nullptr, [&] { *out = new zjai_checkpoint{Checkpoint::parse((const uint8_t*)data, len)}; });
}

extern "C" int32_t zjai_checkpoint_destroy(zjai_checkpoint* ck) {
    delete ck;
    return ZJAI_OK;
}

extern "C" int32_t zjai_checkpoint_counts(const zjai_checkpoint* ck, int32_t* tensors, int32_t* ints, int32_t* lists,
                                          int32_t* packed) {
    if (!ck) return ZJAI_E_INVALID_ARGUMENT;
    if (tensors) *tensors = (int32_t)ck->ck->tensors().size();
    if (ints) *ints = (int32_t)ck->ck->ints().size();
    if (lists) *lists = (int32_t)ck->ck->lists().size();
    if (packed) *packed = ck->ck->packed() ? 1 : 0;
    return ZJAI_OK;
}

extern "C" int32_t zjai_checkpoint_tensor_name(const zjai_checkpoint* ck, int32_t i, char* buf, size_t cap) {
    if (!ck || i < 0 || (size_t)i >= ck->ck->tensors().size()) return ZJAI_E_INVALID_ARGUMENT;
    return guard(nullptr, [&] { copy_name(ck->ck->tensors()[i].name, buf, cap); });
}

extern "C" int32_t zjai_checkpoint_info(const zjai_checkpoint* ck, const char* name, int32_t* dtype, int32_t* rank,
                                        int64_t* shape) {
    return guard(nullptr, [&] {
        const CkTensor& t = tensor_of(ck, name);
        if (t.shape.size() > ZJAI_MAX_RANK) throw Error(ZJAI_E_LIMIT, "tensor rank above 8");
        if (dtype) *dtype = t.dtype;
        if (rank) *rank = (int32_t)t.shape.size();
        if (shape)
            for (size_t k = 0; k < t.shape.size(); ++k) shape[k] = (int64_t)t.shape[k];
    });
}

extern "C" int32_t zjai_checkpoint_read(const zjai_checkpoint* ck, const char* name, void* out, size_t bytes) {
    return guard(nullptr, [&] {
        const CkTensor& t = tensor_of(ck, name);
        const std::vector<uint8_t> b = ck->ck->bytes(t);
        if (b.size() != bytes) throw Error(ZJAI_E_INVALID_ARGUMENT, "output size differs from the tensor's bytes");
        need(out != nullptr || bytes == 0, "null output");
        if (bytes) std::memcpy(out, b.data(), bytes);
    });
}

extern "C" int32_t zjai_checkpoint_read_f32(const zjai_checkpoint* ck, const char* name, float* out, size_t len) {
    return guard(nullptr, [&] {
        const CkTensor& t = tensor_of(ck, name);
        const std::vector<float> v = ck->ck->f32(t);
        if (v.size() != len) throw Error(ZJAI_E_INVALID_ARGUMENT, "output length differs from the tensor's size");
        need(out != nullptr || len == 0, "null output");
        if (len) std::memcpy(out, v.data(), len * 4);
    });
}

extern "C" int32_t zjai_checkpoint_int_at(const zjai_checkpoint* ck, int32_t i, char* buf, size_t cap,
                                          int64_t* value) {
    if (!ck || i < 0 || (size_t)i >= ck->ck->ints().size()) return ZJAI_E_INVALID_ARGUMENT;
    return guard(nullptr, [&] {
        const auto& e = ck->ck->ints()[i];
        if (buf) copy_name(e.first, buf, cap);
        if (value) *value = e.second;
    });
}

extern "C" int32_t zjai_checkpoint_list_at(const zjai_checkpoint* ck, int32_t i, char* buf, size_t cap,
                                           double* values, size_t cap_values, size_t* n) {
    if (!ck || i < 0 || (size_t)i >= ck->ck->lists().size()) return ZJAI_E_INVALID_ARGUMENT;
    return guard(nullptr, [&] {
        const auto& e = ck->ck->lists()[i];
        if (buf) copy_name(e.first, buf, cap);
        if (n) *n = e.second.size();
        if (values) std::copy_n(e.second.begin(), std::min(cap_values, e.second.size()), values);
    });
}

extern "C" int32_t zjai_checkpoint_write_zjm(const zjai_checkpoint* ck, const char* const* names, int32_t n,
                                             int32_t f16, void* out, size_t cap, size_t* len) {
    if (!ck || !len || n < 0 || (n && !names)) return ZJAI_E_INVALID_ARGUMENT;
    return guard(nullptr, [&] {
        std::vector<std::string> nm;
        for (int32_t i = 0; i < n; ++i) {
            need(names[i] != nullptr, "null tensor name");
            nm.push_back(names[i]);
        }
        const std::vector<uint8_t> f = write_zjm(*ck->ck, nm, f16 != 0);
        *len = f.size();
        if (!out) return;
        if (cap < f.size()) throw Error(ZJAI_E_LIMIT, "output buffer too small");
        std::memcpy(out, f.data(), f.size());
    });
}

extern "C" int32_t zjai_bundle_parse(const void* data, size_t len, zjai_bundle** out) {
    if (!out || (!data && len)) return ZJAI_E_INVALID_ARGUMENT;
    *out = nullptr;
    return guard(nullptr, [&] {
        std::unique_ptr<zjai_bundle> b(new zjai_bundle());
        b->b.add((const uint8_t*)data, len);
        *out = b.release();
    });
}

extern "C" int32_t zjai_bundle_add(zjai_bundle* b, const void* data, size_t len) {
    if (!b || (!data && len)) return ZJAI_E_INVALID_ARGUMENT;
    return guard(nullptr, [&] { b->b.add((const uint8_t*)data, len); });
}

extern "C" int32_t zjai_bundle_destroy(zjai_bundle* b) {
    delete b;
    return ZJAI_OK;
}

extern "C" int32_t zjai_bundle_count(const zjai_bundle* b, int32_t* n) {
    if (!b || !n) return ZJAI_E_INVALID_ARGUMENT;
    *n = (int32_t)b->b.paths().size();
    return ZJAI_OK;
}

extern "C" int32_t zjai_bundle_path(const zjai_bundle* b, int32_t i, char* buf, size_t cap) {
    if (!b || i < 0) return ZJAI_E_INVALID_ARGUMENT;
    return guard(nullptr, [&] {
        const std::vector<std::string> p = b->b.paths();
        need((size_t)i < p.size(), "path index out of range");
        copy_name(p[i], buf, cap);
    });
}

extern "C" int32_t zjai_bundle_get(const zjai_bundle* b, const char* rel, const void** data, size_t* len) {
    if (!b || !rel || !data || !len) return ZJAI_E_INVALID_ARGUMENT;
    return guard(nullptr, [&] {
        const auto f = b->b.get(rel);
        if (!f.first) throw Error(ZJAI_E_MODEL, std::string(rel) + ": not in the model bundle");
        *data = f.first;
        *len = f.second;
    });
}

extern "C" int32_t zjai_bundle_notice(const zjai_bundle* b, char* buf, size_t cap, size_t* len) {
    if (!b) return ZJAI_E_INVALID_ARGUMENT;
    return guard(nullptr, [&] {
        const std::string s = b->b.notice();
        if (len) *len = s.size();
        if (buf) copy_name(s, buf, cap);
    });
}

extern "C" int32_t zjai_bundle_write(const char* const* paths, const void* const* files, const size_t* sizes,
                                     int32_t n, const char* notice, int32_t f16, void* out, size_t cap, size_t* len) {
    if (!len || n < 0 || (n && (!paths || !files || !sizes))) return ZJAI_E_INVALID_ARGUMENT;
    return guard(nullptr, [&] {
        std::vector<std::pair<std::string, std::vector<uint8_t>>> fs;
        for (int32_t i = 0; i < n; ++i) {
            need(paths[i] != nullptr && (files[i] != nullptr || sizes[i] == 0), "null file");
            const uint8_t* p = (const uint8_t*)files[i];
            fs.push_back({paths[i], std::vector<uint8_t>(p, p + sizes[i])});
        }
        const std::vector<uint8_t> f = write_bundle(fs, notice ? notice : "", f16 != 0);
        *len = f.size();
        if (!out) return;
        if (cap < f.size()) throw Error(ZJAI_E_LIMIT, "output buffer too small");
        std::memcpy(out, f.data(), f.size());
    });
}

extern "C" int32_t zjai_net_create_from_checkpoint(zjai_ctx* ctx, int32_t op, int32_t component, int32_t precision,
                                                   const zjai_checkpoint* ck, zjai_net** out) {
    if (!ctx || !ck || !out) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        need(precision >= DT_F32 && precision <= DT_BF16, "precision");
        std::vector<std::vector<float>> hold;
        *out = new zjai_net{build_net(ctx->c, op, component, precision, checkpoint_params(*ck->ck, hold))};
    });
}

extern "C" int32_t zjai_latent_model_create_from_checkpoint(zjai_ctx* ctx, int32_t component, int32_t precision,
                                                            const zjai_checkpoint* ck, zjai_net** out) {
    if (!ctx || !ck || !out) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        need(precision >= DT_F32 && precision <= DT_BF16, "precision");
        std::vector<std::vector<float>> hold;
        *out = new zjai_net{build_latent_net(ctx->c, component, precision, checkpoint_params(*ck->ck, hold))};
    });
}

// ------------------------------------------------------------------ analysis transforms
extern "C" int32_t zjai_analysis_create(zjai_ctx* ctx, int32_t op, int32_t component, int32_t precision,
                                        int32_t n_tensors, const char* const* names, const int32_t* ndims,
                                        const int32_t* dims, const float* const* data, zjai_net** out) {
    if (!ctx || !out || n_tensors < 0 || (n_tensors && (!names || !ndims || !dims || !data)))
        return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        need(precision >= DT_F32 && precision <= DT_BF16, "precision");
        *out = new zjai_net{
            build_analysis_net(ctx->c, op, component, precision, params_of(n_tensors, names, ndims, dims, data))};
    });
}

extern "C" int32_t zjai_analysis_create_from_checkpoint(zjai_ctx* ctx, int32_t op, int32_t component,
                                                        int32_t precision, const zjai_checkpoint* ck,
                                                        zjai_net** out) {
    if (!ctx || !ck || !out) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        need(precision >= DT_F32 && precision <= DT_BF16, "precision");
        std::vector<std::vector<float>> hold;
        *out = new zjai_net{build_analysis_net(ctx->c, op, component, precision, checkpoint_params(*ck->ck, hold))};
    });
}

extern "C" int32_t zjai_analysis_forward(zjai_ctx* ctx, const zjai_net* net, const float* x, int32_t c, int32_t h,
                                         int32_t w, int32_t clip, float* y, size_t len) {
    if (!ctx || !net || !x || !y) return ZJAI_E_INVALID_ARGUMENT;
    return guard(ctx, [&] {
        const Net& m = *net->n;
        need(m.kind == NET_ANALYSIS, "not an analysis transform");
        need(c == m.in_ch, "analysis transform: input planes (1 luma, 12 chroma)");
        need(h > 0 && w > 0, "analysis transform: empty picture");
        const int d = m.comp == COMP_Y ? 16 : 8;
        const size_t yn = (size_t)m.chs * ceil_div(h, d) * ceil_div(w, d);
        need(len >= yn, "output buffer too small");
        Context& cx = ctx->c;
        const size_t xn = (size_t)c * h * w;
        float* xdev = (float*)cx.pool.alloc(xn * 4);
        std::shared_ptr<void> keep(xdev, [&cx](void* q) { cx.pool.release(q); });
        ZJAI_HIP(hipMemcpyAsync(xdev, x, xn * 4, hipMemcpyHostToDevice, cx.stream));
        TensorP t = analysis_forward(cx, m, xdev, h, w, clip != 0);
        float* dev = (float*)cx.pool.alloc(yn * 4);
        std::shared_ptr<void> keep2(dev, [&cx](void* q) { cx.pool.release(q); });
        {
            LaunchScope sc(cx, kname("k_nhwc_to_planar", m.dtype), 0.0, (4.0 + dtype_size(m.dtype)) * yn);
            ZJAI_HIP(launch_nhwc_to_planar(t->v, m.dtype, 1, m.chs, t->h, t->w, dev, cx.stream));
        }
        ZJAI_HIP(hipMemcpyAsync(y, dev, yn * 4, hipMemcpyDeviceToHost, cx.stream));
        ZJAI_HIP(hipStreamSynchronize(cx.stream));
    });
}
