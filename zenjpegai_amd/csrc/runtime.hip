// Host runtime: device pool, tensors, weight packing and conv launches.

#include "runtime.h"
#include "checkpoint.h"

#include <cmath>
#include <cstring>

namespace zjai {

// ------------------------------------------------------------------------------------ pool
size_t Pool::bucket(size_t bytes) {
    // 256-byte granularity below 1 MiB, 64 KiB granularity above: tile shapes repeat, so exact
    // sizes recur and blocks are reused without much slack.
    if (bytes <= (1u << 20)) return (bytes + 255) & ~size_t(255);
    return (bytes + 65535) & ~size_t(65535);
}

void* Pool::alloc(size_t bytes) {
    if (faults && faults->take(FAULT_ALLOC)) throw Error(ZJAI_E_LIMIT, "hipMalloc: injected allocation failure");
    const size_t b = bucket(bytes ? bytes : 256);
    auto it = free_.lower_bound(b);
    void* p = nullptr;
    size_t got = 0;
    // Reuse a cached block of the same size, or one at most 1.5x larger.
    if (it != free_.end() && it->first <= b + b / 2) {
        p = it->second;
        got = it->first;
        free_.erase(it);
    } else {
        hipError_t e = hipMalloc(&p, b);
        if (e == hipErrorOutOfMemory) {
            trim();
            e = hipMalloc(&p, b);
        }
        if (e != hipSuccess)
            throw Error(e == hipErrorOutOfMemory ? ZJAI_E_LIMIT : ZJAI_E_DEVICE,
                        std::string("hipMalloc: ") + hipGetErrorString(e));
        got = b;
        cached_ += b;
    }
    live_[p] = got;
    in_use_ += got;
    if (in_use_ > peak_) peak_ = in_use_;
    return p;
}

void Pool::release(void* p) {
    auto it = live_.find(p);
    if (it == live_.end()) return;
    in_use_ -= it->second;
    free_.emplace(it->second, p);
    live_.erase(it);
}

void Pool::trim() {
    (void)hipDeviceSynchronize();
    for (auto& kv : free_) {
        (void)hipFree(kv.second);
        cached_ -= kv.first;
    }
    free_.clear();
}

void Pool::surrender(std::vector<void*>& out) {
    for (auto& kv : free_) {
        out.push_back(kv.second);
        cached_ -= kv.first;
    }
    free_.clear();
}

Pool::~Pool() {
    for (auto& kv : free_) (void)hipFree(kv.second);
    for (auto& kv : live_) (void)hipFree(kv.first);
}

// --------------------------------------------------------------------------------- tensors
TensorP Context::alloc(int n, int c, int h, int w, int dtype) {
    if (n <= 0 || n > MAXB || c <= 0 || h < 0 || w < 0) throw Error(ZJAI_E_INVALID_ARGUMENT, "tensor: bad shape");
    auto t = std::make_shared<Tensor>();
    t->ctx = this;
    t->dtype = dtype;
    t->n = n;
    t->c = c;
    t->h = h;
    t->w = w;
    t->v.cs = round_up(c, 8);
    t->v.row = (long long)w * t->v.cs;
    t->v.bstride = (long long)h * t->v.row;
    t->v.c_off = 0;
    const size_t bytes = (size_t)n * (size_t)t->v.bstride * dtype_size(dtype);
    void* p = pool.alloc(bytes);
    std::shared_ptr<Pool> owner = pool_owner;
    t->keep = std::shared_ptr<void>(p, [owner](void* q) { owner->release(q); });
    t->base = p;
    t->v.p = p;
    return t;
}

void Context::check_stop() {
    if (top().stop) throw Error(ZJAI_E_CANCELLED, "cancelled");
}

Context& Context::lane(int i) {
    if (root) return root->lane(i);
    while ((int)lanes.size() <= i) {
        auto l = std::make_unique<Context>();
        l->root = this;
        l->device = device;
        l->faults = faults;
        l->pool.faults = faults;
        ZJAI_HIP(hipSetDevice(device));
        ZJAI_HIP(hipStreamCreateWithFlags(&l->stream, hipStreamNonBlocking));
        l->owns_stream = true;
        lanes.push_back(std::move(l));
    }
    return *lanes[i];
}

hipEvent_t Context::take_event() {
    if (root) return root->take_event();
    if (ev_used == ev_pool.size()) {
        hipEvent_t e;
        ZJAI_HIP(hipEventCreate(&e));
        ev_pool.push_back(e);
    }
    return ev_pool[ev_used++];
}

Context::~Context() {
    lanes.clear();
    if (owns_stream && stream) {
        (void)hipStreamSynchronize(stream);
        (void)hipStreamDestroy(stream);
    }
    for (hipEvent_t e : ev_pool) (void)hipEventDestroy(e);
    if (range_slots) (void)hipFree(range_slots);
}

void range_slots_init(Context& ctx) {
    if (ctx.range_slots || !(ctx.top().flags & ZJAI_CTX_COUNT_F16_RANGE)) return;
    ZJAI_HIP(hipMalloc(&ctx.range_slots, sizeof(unsigned long long) * RANGE_SLOTS));
    ZJAI_HIP(launch_zero(ctx.range_slots, sizeof(unsigned long long) * RANGE_SLOTS, ctx.stream));
}

void count_f16_range(Context& ctx, const Tensor& t) {
    if (t.dtype != DT_F16 || !(ctx.top().flags & ZJAI_CTX_COUNT_F16_RANGE)) return;
    range_slots_init(ctx);
    LaunchScope sc(ctx, "k_count_f16_nonfinite", 0.0, 2.0 * t.n * t.c * t.h * t.w);
    ZJAI_HIP(launch_count_f16_nonfinite(t.v, t.n, t.c, t.h, t.w, ctx.range_slots, RANGE_SLOTS, ctx.stream));
}

unsigned long long f16_range_total(Context& root) {
    unsigned long long total = 0;
    std::vector<unsigned long long> h(RANGE_SLOTS);
    auto add = [&](Context& c) {
        if (!c.range_slots) return;
        ZJAI_HIP(hipStreamSynchronize(c.stream));
        ZJAI_HIP(hipMemcpy(h.data(), c.range_slots, sizeof(unsigned long long) * RANGE_SLOTS, hipMemcpyDeviceToHost));
        for (unsigned long long v : h) total += v;
    };
    add(root);
    for (auto& l : root.lanes) add(*l);
    return total;
}

LaunchScope::LaunchScope(Context& c, const std::string& name, double flops, double bytes) : c_(c) {
    Context& t = c_.top();
    if (t.faults->take(FAULT_LAUNCH)) throw Error(ZJAI_E_DEVICE, name + ": injected launch failure");
    ++t.launches;
    if (!t.profiling) return;
    ProfRec r;
    r.name = name;
    r.flops = flops;
    r.bytes = bytes;
    r.a = t.take_event();
    r.b = t.take_event();
    ZJAI_HIP(hipEventRecord(r.a, c_.stream));
    idx_ = (long)t.prof.size();
    t.prof.push_back(r);
}

LaunchScope::~LaunchScope() {
    if (idx_ >= 0) (void)hipEventRecord(c_.top().prof[idx_].b, c_.stream);
}

TensorP crop_view(const TensorP& t, int h, int w) {
    if (h > t->h || w > t->w || h < 0 || w < 0)
        throw Error(ZJAI_E_INVALID_ARGUMENT, "crop larger than tensor");
    if (h == t->h && w == t->w) return t;
    auto v = std::make_shared<Tensor>(*t);
    v->h = h;
    v->w = w;
    return v;
}

TensorP channel_view(const TensorP& t, int c0, int n) {
    if (c0 < 0 || n <= 0 || c0 + n > t->c) throw Error(ZJAI_E_INVALID_ARGUMENT, "channel range");
    auto v = std::make_shared<Tensor>(*t);
    v->c = n;
    v->v.c_off = t->v.c_off + c0;
    return v;
}

// ------------------------------------------------------------------------ weight conversion
// f32 -> bf16 bits, round to nearest even (NaN kept quiet).
static uint16_t f32_to_bf16_bits(float v) {
    uint32_t b;
    std::memcpy(&b, &v, 4);
    if ((b & 0x7fffffff) > 0x7f800000) return (uint16_t)((b >> 16) | 0x40);
    const uint32_t r = b + 0x7fff + ((b >> 16) & 1);
    return (uint16_t)(r >> 16);
}

// The f32 value of a storage-dtype weight (f16 / bf16 upcasts are exact).
static float storage_value(float v, int dtype) {
    if (dtype == DT_F32) return v;
    uint32_t b;
    if (dtype == DT_BF16) {
        b = (uint32_t)f32_to_bf16_bits(v) << 16;
    } else {
        const uint32_t h = f32_to_f16_bits(v), sign = (h & 0x8000u) << 16;
        const uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff;
        if (e == 31) {
            b = sign | 0x7f800000u | (m << 13);
        } else if (e) {
            b = sign | ((e + 112) << 23) | (m << 13);
        } else if (!m) {
            b = sign;
        } else {  // subnormal half: normalise
            int sh = 0;
            uint32_t mm = m;
            while (!(mm & 0x400)) { mm <<= 1; ++sh; }
            b = sign | ((uint32_t)(113 - sh) << 23) | ((mm & 0x3ff) << 13);
        }
    }
    float f;
    std::memcpy(&f, &b, 4);
    return f;
}

// Converts an f32 staging vector to the storage dtype and uploads it.
static void* upload_as(Context& ctx, const std::vector<float>& host, int dtype, size_t* bytes_out,
                       size_t* total) {
    const size_t n = host.size();
    void* dev = nullptr;
    if (dtype == DT_F32) {
        ZJAI_HIP(hipMalloc(&dev, n * 4));
        ZJAI_HIP(hipMemcpy(dev, host.data(), n * 4, hipMemcpyHostToDevice));
        *bytes_out = n * 4;
    } else {
        std::vector<uint16_t> h(n);
        for (size_t i = 0; i < n; ++i)
            h[i] = dtype == DT_F16 ? f32_to_f16_bits(host[i]) : f32_to_bf16_bits(host[i]);
        ZJAI_HIP(hipMalloc(&dev, n * 2));
        ZJAI_HIP(hipMemcpy(dev, h.data(), n * 2, hipMemcpyHostToDevice));
        *bytes_out = n * 2;
    }
    *total += *bytes_out;
    (void)ctx;
    return dev;
}

static float* upload_f32(const float* p, size_t n, size_t* total) {
    float* dev = nullptr;
    *total += n * 4;
    ZJAI_HIP(hipMalloc(&dev, n * 4));
    ZJAI_HIP(hipMemcpy(dev, p, n * 4, hipMemcpyHostToDevice));
    return dev;
}

Layer::~Layer() {
    if (wpk) (void)hipFree(wpk);
    if (bias) (void)hipFree(bias);
    if (dw_w) (void)hipFree(dw_w);
    if (w_f32) (void)hipFree(w_f32);
    if (wn) (void)hipFree(wn);
    if (wm16) (void)hipFree(wm16);
    if (wpk_m) (void)hipFree(wpk_m);
    if (wpk32) (void)hipFree(wpk32);
}

void Layer::out_size(int h, int w, int* oh, int* ow) const {
    if (transposed) {
        *oh = (h - 1) * stride + k + out_pad - 2 * pad;
        *ow = (w - 1) * stride + k + out_pad - 2 * pad;
    } else {
        *oh = (h + extra[0] + extra[2] + 2 * pad_h - kh) / stride + 1;
        *ow = (w + extra[1] + extra[3] + 2 * pad_w - kw) / stride + 1;
    }
}

// Tile shape of a layer: narrow groups / outputs take 16- or 32-channel tiles; dense stride-1
// 3x3 layers take the 8-wave 64-channel x 16-row tile (two waves per SIMD from one workgroup hide
// each other's LDS and barrier waits: +2-3 % on the config-5 picture in every precision); fp32
// 1x1 layers with >= 256 outputs the 8-wave 128-channel x 8-row tile (+2 % in fp32).
TileCfg conv_tile_cfg(int cout_g, int kind, int dtype) {
    if (cout_g <= 16) return TileCfg{1, 4, 1, 2};
    if (cout_g <= 32) return TileCfg{1, 4, 2, 2};
    if (kind == CK_3x3) return TileCfg{2, 4, 2, 4};
    if (kind == CK_1x1 && dtype == DT_F32 && cout_g >= 256 && cout_g % 128 == 0) return TileCfg{4, 2, 2, 4};
    return TileCfg{2, 2, 2, 4};
}

LayerP make_conv(Context& ctx, int cin, int cout, int kh, int kw, int stride, int pad_h,
                 int pad_w, int groups, const float* weight, const float* bias,
                 const int extra[4], int dtype, bool keep_f32) {
    if (groups <= 0 || cin <= 0 || cout <= 0 || cin % groups || cout % groups || stride <= 0 ||
        kh <= 0 || kw <= 0 || pad_h < 0 || pad_w < 0)
        throw Error(ZJAI_E_MODEL, "conv2d: inconsistent channel/group/kernel configuration");
    if (dtype < DT_F32 || dtype > DT_BF16) throw Error(ZJAI_E_INVALID_ARGUMENT, "precision");
    if (!weight) throw Error(ZJAI_E_INVALID_ARGUMENT, "conv2d: null weight");
    auto L = std::make_shared<Layer>();
    L->cin = cin; L->cout = cout; L->kh = kh; L->kw = kw; L->stride = stride;
    L->pad_h = pad_h; L->pad_w = pad_w; L->groups = groups; L->dtype = dtype;
    if (extra) for (int i = 0; i < 4; ++i) {
        if (extra[i] < 0) throw Error(ZJAI_E_INVALID_ARGUMENT, "extra pad");
        L->extra[i] = extra[i];
    }
    const int cin_g = cin / groups, cout_g = cout / groups;
    const bool no_extra = !(L->extra[0] | L->extra[1] | L->extra[2] | L->extra[3]);
    if (groups == cin && groups == cout && kh == 3 && kw == 3 && stride == 1 && pad_h == 1 &&
        pad_w == 1 && no_extra) {
        if (cin % 4) throw Error(ZJAI_E_UNSUPPORTED, "depthwise: channels not a multiple of 4");
        L->depthwise = true;
        std::vector<float> t((size_t)9 * cin);
        for (int c = 0; c < cin; ++c)
            for (int k = 0; k < 9; ++k) t[(size_t)k * cin + c] = weight[(size_t)c * 9 + k];
        L->dw_w = upload_f32(t.data(), t.size(), &L->dev_bytes);
        if (bias) L->bias = upload_f32(bias, cout, &L->dev_bytes);
        return L;
    }
    if (kh == 1 && kw == 1 && stride == 1) L->kind = CK_1x1;
    else if (kh == 2 && kw == 2 && stride == 1) L->kind = CK_2x2;
    else if (kh == 3 && kw == 3 && stride == 1) L->kind = CK_3x3;
    else if (kh == 3 && kw == 3 && stride == 2) L->kind = CK_3x3_S2;
    else throw Error(ZJAI_E_UNSUPPORTED, "conv2d: kernel geometry without a HIP kernel");
    const int vec = 16 / dtype_size(dtype);
    if (cin_g % vec) throw Error(ZJAI_E_UNSUPPORTED, "conv2d: channels per group not vector aligned");
    L->cfg = conv_tile_cfg(cout_g, L->kind, dtype);
    const int NB = L->cfg.wc * L->cfg.cf;
    const int CK = 64 / dtype_size(dtype);
    const int T = kh * kw;
    L->nblk_g = round_up(ceil_div(cout_g, 16), NB);
    L->nchunks = ceil_div(cin_g, CK);
    std::vector<float> pk((size_t)groups * L->nchunks * L->nblk_g * T * 16 * CK, 0.0f);
    for (int g = 0; g < groups; ++g)
        for (int ocl = 0; ocl < cout_g; ++ocl)
            for (int icl = 0; icl < cin_g; ++icl)
                for (int ky = 0; ky < kh; ++ky)
                    for (int kx = 0; kx < kw; ++kx) {
                        const int ch = icl / CK, kk = icl % CK, nb = ocl / 16, r = ocl % 16;
                        const int t = ky * kw + kx;
                        const size_t dst = ((((size_t)g * L->nchunks + ch) * L->nblk_g + nb) * T + t) * 16 * CK +
                                           (size_t)r * CK + kk;
                        pk[dst] = weight[(((size_t)(g * cout_g + ocl) * cin_g + icl) * kh + ky) * kw + kx];
                    }
    L->wpk = upload_as(ctx, pk, dtype, &L->wpk_bytes, &L->dev_bytes);
    if (dtype != DT_F32 && L->kind == CK_3x3 && groups == 1 && (cin == 64 || cin == 128) && cout % 64 == 0 && no_extra &&
        pad_h == 1 && pad_w == 1) {
        // conv3x3_m32's packing: [cin / 16][cout / mt][tap][channel half][mt][8].
        const int mt = cout % 128 == 0 ? 128 : 64, nmt = cout / mt;
        std::vector<float> p32((size_t)cin * cout * 9);
        for (int oc = 0; oc < cout; ++oc)
            for (int ic = 0; ic < cin; ++ic)
                for (int t = 0; t < 9; ++t)
                    p32[(((((size_t)(ic / 16) * nmt + oc / mt) * 9 + t) * 2 + (ic % 16) / 8) * mt + oc % mt) * 8 +
                        ic % 8] = weight[((size_t)oc * cin + ic) * 9 + t];
        size_t bytes = 0;
        L->wpk32 = upload_as(ctx, p32, dtype, &bytes, &L->dev_bytes);
        L->mt32 = mt;
    }
    if (bias) L->bias = upload_f32(bias, cout, &L->dev_bytes);
    if (keep_f32 && L->kind == CK_1x1 && groups == 1) L->w_f32 = upload_f32(weight, (size_t)cout * cin, &L->dev_bytes);
    return L;
}

LayerP make_conv_transpose(Context& ctx, int cin, int cout, int k, int stride, int pad,
                           int out_pad, const float* weight, const float* bias, int dtype) {
    if (stride <= 0 || k <= 0 || pad < 0 || pad >= k || out_pad < 0 || out_pad >= stride ||
        cin <= 0 || cout <= 0)
        throw Error(ZJAI_E_MODEL, "conv_transpose2d: unsupported geometry");
    if (dtype < DT_F32 || dtype > DT_BF16) throw Error(ZJAI_E_INVALID_ARGUMENT, "precision");
    if (!weight) throw Error(ZJAI_E_INVALID_ARGUMENT, "conv_transpose2d: null weight");
    if (stride != 2) throw Error(ZJAI_E_UNSUPPORTED, "conv_transpose2d: only stride 2 has a HIP kernel");
    auto L = std::make_shared<Layer>();
    L->transposed = true;
    L->cin = cin; L->cout = cout; L->k = k; L->stride = stride; L->pad = pad;
    L->out_pad = out_pad; L->dtype = dtype; L->groups = 1; L->kind = CK_T3;
    // Per output phase (py, px): the taps whose stride parity reaches it, ky then kx ascending
    // (reference src/nn/reference.rs:175-199), with their input row/col offsets.
    int ky_list[2][4], nky[2] = {0, 0}, dy_list[2][4];
    for (int pp = 0; pp < 2; ++pp)
        for (int kk = 0; kk < k; ++kk) {
            const int d = pp + pad - kk;
            if (((d % 2) + 2) % 2) continue;
            const int off = (d >= 0 ? d / 2 : -((-d) / 2)) + 1;
            if (off < 0 || off > 2 || nky[pp] >= 2)
                throw Error(ZJAI_E_UNSUPPORTED, "conv_transpose2d: tap reach beyond the 3x3 halo");
            ky_list[pp][nky[pp]] = kk;
            dy_list[pp][nky[pp]] = off;
            ++nky[pp];
        }
    for (int ph = 0; ph < 4; ++ph) {
        const int py = ph >> 1, px = ph & 1;
        int n = 0;
        for (int a = 0; a < nky[py]; ++a)
            for (int b = 0; b < nky[px]; ++b) {
                L->tap_dy[ph][n] = dy_list[py][a];
                L->tap_dx[ph][n] = dy_list[px][b];
                ++n;
            }
        L->ntaps[ph] = n;
    }
    const int vec = 16 / dtype_size(dtype);
    if (cin % vec) throw Error(ZJAI_E_UNSUPPORTED, "conv_transpose2d: channels not vector aligned");
    L->cfg = conv_tile_cfg(cout, CK_T3, dtype);
    const int NB = L->cfg.wc * L->cfg.cf;
    const int CK = 64 / dtype_size(dtype);
    L->nblk_g = round_up(ceil_div(cout, 16), NB);
    L->nchunks = ceil_div(cin, CK);
    L->phase_stride = (long long)L->nchunks * L->nblk_g * 4 * 16 * CK;
    std::vector<float> pk((size_t)4 * L->phase_stride, 0.0f);
    for (int ph = 0; ph < 4; ++ph) {
        const int py = ph >> 1, px = ph & 1;
        int t = 0;
        for (int a = 0; a < nky[py]; ++a)
            for (int b = 0; b < nky[px]; ++b, ++t) {
                const int ky = ky_list[py][a], kx = ky_list[px][b];
                for (int oc = 0; oc < cout; ++oc)
                    for (int ic = 0; ic < cin; ++ic) {
                        const int ch = ic / CK, kk = ic % CK, nb = oc / 16, r = oc % 16;
                        const size_t dst = (size_t)ph * L->phase_stride +
                                           ((((size_t)ch * L->nblk_g + nb) * 4 + t) * 16 + r) * CK + kk;
                        pk[dst] = weight[(((size_t)ic * cout + oc) * k + ky) * k + kx];
                    }
            }
    }
    L->wpk = upload_as(ctx, pk, dtype, &L->wpk_bytes, &L->dev_bytes);
    if (bias) L->bias = upload_f32(bias, cout, &L->dev_bytes);
    if (k == 3 && cout > 8 && conv_tr_merged_taps_supported(L->ntaps) && L->nblk_g % TR_MERGED_NB == 0) {
        // All four phases per workgroup (launch_conv_tr_merged): the nine taps side by side per
        // K chunk and block, phase by phase, each phase's taps in its table order.
        std::vector<float> pm((size_t)L->nchunks * L->nblk_g * TR_MERGED_TAPS * 16 * CK, 0.0f);
        for (int ch = 0; ch < L->nchunks; ++ch)
            for (int nb = 0; nb < L->nblk_g; ++nb) {
                int e = 0;
                for (int ph = 0; ph < 4; ++ph)
                    for (int t = 0; t < L->ntaps[ph]; ++t, ++e) {
                        const float* src = pk.data() + (size_t)ph * L->phase_stride +
                                           (((size_t)ch * L->nblk_g + nb) * 4 + t) * 16 * CK;
                        float* dst = pm.data() + (((size_t)ch * L->nblk_g + nb) * TR_MERGED_TAPS + e) * 16 * CK;
                        if (dtype != DT_F32) {
                            // 16-bit: 16-byte unit q of row r at q ^ 2 (bit 2 of r), the layout
                            // conv_tr_merged's fragment reads expect (conflict-free ds_read_b128).
                            for (int r = 0; r < 16; ++r)
                                for (int q = 0; q < 4; ++q)
                                    std::copy(src + r * CK + q * (CK / 4), src + r * CK + (q + 1) * (CK / 4),
                                              dst + r * CK + (q ^ ((r & 4) >> 1)) * (CK / 4));
                        } else {
                            std::copy(src, src + 16 * CK, dst);
                        }
                    }
            }
        L->wpk_m = upload_as(ctx, pm, dtype, &L->wpk_m_bytes, &L->dev_bytes);
    }
    if (cout <= 8) {
        // Narrow layers run on the vector ALUs (launch_convT_narrow) from an f32 copy of the
        // storage-rounded weights, [cin][phase][tap][coutp].
        L->coutp = cout <= 1 ? 1 : cout <= 2 ? 2 : cout <= 4 ? 4 : 8;
        std::vector<float> wn((size_t)16 * cin * L->coutp, 0.0f);
        for (int ph = 0; ph < 4; ++ph) {
            const int py = ph >> 1, px = ph & 1;
            int t = 0;
            for (int a = 0; a < nky[py]; ++a)
                for (int b = 0; b < nky[px]; ++b, ++t) {
                    const int ky = ky_list[py][a], kx = ky_list[px][b];
                    for (int ic = 0; ic < cin; ++ic)
                        for (int oc = 0; oc < cout; ++oc)
                            wn[((size_t)ic * 16 + ph * 4 + t) * L->coutp + oc] =
                                storage_value(weight[(((size_t)ic * cout + oc) * k + ky) * k + kx], dtype);
                }
        }
        L->wn = upload_f32(wn.data(), wn.size(), &L->dev_bytes);
        if (dtype != DT_F32 && k == 3 && (cin == 64 || cin == 128)) {
            // The MFMA form (launch_convT3_mfma): row R = phase * coutp + output of 16-row block
            // R / 16, K = (neighbour, input channel); tap t of phase ph reads input pixel
            // (y' + tap_dy - 1, x' + tap_dx - 1), i.e. neighbour 2 (tap_dy - 1) + (tap_dx - 1)
            // when both offsets are 1 or 2 (the 3x3 / padding-1 tables).
            const int mbn = (4 * L->coutp + 15) / 16;
            std::vector<float> wm((size_t)(cin / 32) * 4 * mbn * 16 * 32, 0.0f);
            bool ok = true;
            for (int ph = 0; ph < 4; ++ph)
                for (int t = 0; t < L->ntaps[ph]; ++t) {
                    const int dy = L->tap_dy[ph][t], dx = L->tap_dx[ph][t];
                    if (dy < 1 || dy > 2 || dx < 1 || dx > 2) ok = false;
                    if (!ok) continue;
                    const int n = 2 * (dy - 1) + (dx - 1);
                    for (int oc = 0; oc < cout; ++oc) {
                        const int R = ph * L->coutp + oc, mb = R / 16, row = R % 16;
                        for (int ic = 0; ic < cin; ++ic)
                            wm[((((size_t)(ic / 32) * 4 + n) * mbn + mb) * 16 + row) * 32 + ic % 32] =
                                wn[((size_t)ic * 16 + ph * 4 + t) * L->coutp + oc];
                    }
                }
            if (ok) L->wm16 = upload_as(ctx, wm, dtype, &L->wm16_bytes, &L->dev_bytes);
        }
    }
    return L;
}

// ------------------------------------------------------------------------------ conv launch
// The kernel's name as profilers print it: conv_igemm<T, KH, KW, S, TR, WC, WP, CF, PF>.
// Launch-time tile shape of a dense layer. The layer's own shape (64 channels x 16 or 8 rows)
// suits large maps; on small ones its grid leaves most of the 256 CUs idle while each workgroup
// walks the whole K loop, so narrower tiles (32 or 16 channels x 8 rows; the weights are packed
// per 16-channel block, so any of them reads the same packing) take over below a workgroup
// count. Every shape sums each output in the same order (bias, then K chunk by chunk, tap by
// tap), so the choice never changes a result. Thresholds from the per-layer sweep (fp32 /
// 16-bit): 3x3 192 -> 192 at 40 x 80 runs 112 -> 44 us / 25 -> 17 us; at 256^2 and 128 channels
// (512 tiles) the 16-row tile stays fastest.
static TileCfg launch_tile_cfg(const Layer& L, int N, int OH, int OW) {
    const TileCfg c = L.cfg;
    if (L.groups != 1) return c;
    const long long nt4 = L.nblk_g / 4;
    if (L.kind == CK_3x3 && c.wc == 2 && c.wp == 4 && c.cf == 2 && c.pf == 4) {
        const long long w0 = (long long)((OW + 15) / 16) * ((OH + 15) / 16) * N * nt4;
        if (L.dtype == DT_F32) return w0 < 256 ? TileCfg{1, 4, 1, 2} : c;
        return w0 < 64 ? TileCfg{1, 4, 1, 2} : w0 < 256 ? TileCfg{1, 4, 2, 2} : c;
    }
    if (L.kind == CK_3x3_S2 && c.wc == 2 && c.wp == 2 && c.cf == 2 && c.pf == 4) {
        const long long w0 = (long long)((OW + 15) / 16) * ((OH + 7) / 8) * N * nt4;
        if (w0 < 128) return TileCfg{1, 4, 1, 2};
        // 16-bit: 128-channel tiles (8 waves) share each staged halo between twice the outputs.
        if (L.dtype != DT_F32 && L.nblk_g % 8 == 0 && w0 >= 512) return TileCfg{4, 2, 2, 4};
        return c;
    }
    if (L.kind == CK_2x2 && c.wc == 2 && c.wp == 2 && c.cf == 2 && c.pf == 4) {
        // The SOP / BOP upsampling convs (2x2 + pixel shuffle) run on the latent grid or twice
        // it, where the default tile leaves CUs idle: 160 -> 256 at 64^2 has 128 tiles.
        const long long w0 = (long long)((OW + 15) / 16) * ((OH + 7) / 8) * N * nt4;
        return w0 < 256 ? TileCfg{1, 4, 1, 2} : w0 < 512 ? TileCfg{1, 4, 2, 2} : c;
    }
    if (L.kind == CK_T3 && L.wpk_m && c.wc == 2 && c.wp == 2 && c.cf == 2 && c.pf == 4) {
        // 3x3 transposed layers whose merged grid is small (see convT_merged_fills).
        const long long wm = (long long)(((OW + 1) / 2 + 15) / 16) * (((OH + 1) / 2 + 15) / 16) * N * nt4;
        return wm < 64 ? TileCfg{1, 4, 1, 2} : wm < 256 ? TileCfg{1, 4, 2, 2} : c;
    }
    return c;
}

// Transposed 3x3 layers take the merged four-phase kernel when its grid (16 x 16 phase positions
// x 64 channels per workgroup) has at least 256 workgroups, else the phase-split kernel on a
// narrow tile: 192 -> 192 from 40^2 runs 119 -> 38 us (fp32), from 80^2 125 -> 88 us; from 160^2
// the merged kernel is faster (257 vs 304 us).
static bool convT_merged_fills(const Layer& L, int N, int OH, int OW) {
    const long long wm = (long long)(((OW + 1) / 2 + 15) / 16) * (((OH + 1) / 2 + 15) / 16) * N *
                         (L.nblk_g / TR_MERGED_NB);
    return wm >= 256;
}

std::string conv_kernel_name(int kind, int dtype, TileCfg c) {
    static const char* geo[] = {"1, 1, 1, false", "2, 2, 1, false", "3, 3, 1, false", "3, 3, 2, false",
                                "3, 3, 1, true"};
    static const char* ty[] = {"float", "_Float16", "__bf16"};
    char buf[128];
    const bool dma = dtype == DT_F32 && c.cf == 2 && c.pf == 4 &&
                     ((c.wc == 2 && (c.wp == 2 || c.wp == 4)) || (c.wc == 4 && c.wp == 2));
    if (dma)  // the fp32 dense shapes run conv_dma_f32 (conv.hip)
        snprintf(buf, sizeof buf, "conv_dma_f32<%s, %d, %d, %d, %d>", geo[kind], c.wc, c.wp, c.cf, c.pf);
    else
        snprintf(buf, sizeof buf, "conv_igemm<%s, %s, %d, %d, %d, %d>", ty[dtype], geo[kind], c.wc, c.wp, c.cf, c.pf);
    return buf;
}
static View view_of(const Tensor* t) { return t ? t->v : View{nullptr, 0, 0, 0, 0}; }

static TensorP conv_forward_impl(Context& ctx, const Layer& L, const TensorP& x, const Epilogue& e,
                                 const TensorP& dst, const PlaneOut* plane) {
    if (x->c != L.cin) throw Error(ZJAI_E_INVALID_ARGUMENT, "conv: input channel count mismatch");
    if (x->dtype != L.dtype) throw Error(ZJAI_E_INVALID_ARGUMENT, "conv: input precision mismatch");
    const int N = x->n;
    int OH, OW;
    L.out_size(x->h, x->w, &OH, &OW);
    if (OH <= 0 || OW <= 0) throw Error(ZJAI_E_INVALID_ARGUMENT, "conv: input smaller than the kernel");
    const int ps = e.ps > 0 ? e.ps : 1;
    if (L.cout % (ps * ps)) throw Error(ZJAI_E_INVALID_ARGUMENT, "pixel_shuffle: channels not divisible by r^2");
    for (const Tensor* r : {e.r1, e.r2}) {
        if (!r) continue;
        if (r->n != N || r->c != L.cout || r->h != OH || r->w != OW || r->dtype != L.dtype)
            throw Error(ZJAI_E_INVALID_ARGUMENT, "conv epilogue: residual shape differs");
    }
    if ((e.res != RES_NONE && !e.r1) || (e.res == RES_CAB && !e.r2))
        throw Error(ZJAI_E_INVALID_ARGUMENT, "conv epilogue: missing residual");
    TensorP y;
    if (!plane) {
        if (dst) {
            if (dst->n != N || dst->c != L.cout / (ps * ps) || dst->h != OH * ps || dst->w != OW * ps ||
                dst->dtype != L.dtype)
                throw Error(ZJAI_E_INVALID_ARGUMENT, "conv: destination shape differs");
            y = dst;
        } else {
            y = ctx.alloc(N, L.cout / (ps * ps), OH * ps, OW * ps, L.dtype);
        }
    }
    const double es = dtype_size(L.dtype);
    if (L.depthwise) {
        if (e.act || e.res || ps != 1 || e.relu6_in || plane || e.w_batch)
            throw Error(ZJAI_E_UNSUPPORTED, "depthwise: fused epilogue");
        LaunchScope sc(ctx, kname("k_depthwise3x3", L.dtype), 2.0 * 9 * N * L.cin * x->h * x->w, 2.0 * es * N * L.cin * x->h * x->w);
        ZJAI_HIP(launch_depthwise3x3(x->v, y->v, L.dtype, N, L.cin, x->h, x->w, L.dw_w, L.bias, 0, ctx.stream));
        return y;
    }
    ConvParams p{};
    p.x = x->v;
    p.H = x->h;
    p.W = x->w;
    p.N = N;
    p.OH = OH;
    p.OW = OW;
    p.y = y ? y->v : View{nullptr, 0, 0, 0, 0};
    p.w = e.w_batch ? e.w_batch : L.wpk;
    p.w_bstride = e.w_batch ? e.w_bstride : 0;
    p.bias = L.bias;
    p.cin_g = L.cin / L.groups;
    p.cout_g = L.cout / L.groups;
    p.groups = L.groups;
    p.nchunks = L.nchunks;
    p.nblk_g = L.nblk_g;
    p.ntiles = L.groups * L.nblk_g / (L.cfg.wc * L.cfg.cf);
    p.phase_stride = L.phase_stride;
    p.pad_t = L.pad_h + L.extra[0];
    p.pad_l = L.pad_w + L.extra[1];
    p.relu6_in = e.relu6_in;
    p.act = e.act;
    p.res = e.res;
    p.r1 = view_of(e.r1);
    p.r2 = view_of(e.r2);
    p.ps = ps;
    if (plane) {
        p.out_mode = OUT_PLANE;
        p.plane = plane->plane;
        p.pl_row = plane->row;
        p.pl_cstride = plane->cstride;
        p.sv = plane->sv;
        p.sh = plane->sh;
        p.denorm = plane->denorm;
        p.bit_depth = plane->bit_depth;
        for (int b = 0; b < MAXB; ++b) {
            p.win_y0[b] = plane->win_y0[b];
            p.win_x0[b] = plane->win_x0[b];
            p.win_h[b] = plane->win_h[b];
            p.win_w[b] = plane->win_w[b];
            p.dst_y0[b] = plane->dst_y0[b];
            p.dst_x0[b] = plane->dst_x0[b];
        }
    } else {
        p.out_mode = OUT_NHWC;
        p.sv = p.sh = 1;
    }
    for (int ph = 0; ph < 4; ++ph) {
        p.ntaps[ph] = L.ntaps[ph];
        for (int t = 0; t < 4; ++t) {
            p.tap_dy[ph][t] = L.tap_dy[ph][t];
            p.tap_dx[ph][t] = L.tap_dx[ph][t];
        }
    }
    // Algorithmic work: every tap of every output (padding taps included); compulsory bytes:
    // input, output, weights and residual reads once each.
    double macs;
    if (L.transposed) {
        double taps = 0.0;
        for (int ph = 0; ph < 4; ++ph)
            taps += (double)((OH - (ph >> 1) + 1) / 2) * ((OW - (ph & 1) + 1) / 2) * L.ntaps[ph];
        macs = taps * L.cout * L.cin;
    } else {
        macs = (double)OH * OW * L.cout * (L.cin / L.groups) * L.kh * L.kw;
    }
    macs *= N;
    double bytes = es * N * ((double)L.cin * x->h * x->w + (double)L.cout * OH * OW) +
                   (double)L.wpk_bytes * (e.w_batch ? N : 1);
    if (e.r1) bytes += es * N * (double)L.cout * OH * OW;
    if (e.r2) bytes += es * N * (double)L.cout * OH * OW;
    if (L.wn && !e.w_batch && L.wm16 && !(ctx.top().flags & ZJAI_CTX_VALU_NARROW_CONVT) &&
        convT_mfma_k3(L.dtype, p, L.cin)) {
        static const char* ty[] = {"float", "_Float16", "__bf16"};
        char name[64];
        snprintf(name, sizeof name, "k_convT3_mfma<%s, %d>", ty[L.dtype], L.coutp);
        LaunchScope sc(ctx, name, 2.0 * macs, bytes);
        ZJAI_HIP(launch_convT3_mfma(L.dtype, L.coutp, p, L.wm16, L.cin, ctx.stream));
        return y;
    }
    if (L.wn && !e.w_batch) {
        static const char* ty[] = {"float", "_Float16", "__bf16"};
        char name[64];
        snprintf(name, sizeof name, "%s<%s, %d>", convT_narrow_k3(L.dtype, p, L.cin) ? "k_convT3_narrow" : "k_convT_narrow",
                 ty[L.dtype], L.coutp);
        LaunchScope sc(ctx, name, 2.0 * macs, bytes);
        ZJAI_HIP(launch_convT_narrow(L.dtype, L.coutp, p, L.wn, L.cin, ctx.stream));
        return y;
    }
    if (L.wpk_m && !e.w_batch && !plane && ps == 1 && !e.relu6_in && convT_merged_fills(L, N, OH, OW) &&
        !(ctx.top().flags & ZJAI_CTX_PHASE_SPLIT_CONVT)) {
        static const char* ty[] = {"float", "_Float16", "__bf16"};
        p.w = L.wpk_m;
        p.ntiles = L.nblk_g / TR_MERGED_NB;
        LaunchScope sc(ctx,
                       std::string("conv_tr_merged<") + ty[L.dtype] + ", " + std::to_string(L.ntaps[0]) + ", " +
                           std::to_string(L.ntaps[1]) + ", " + std::to_string(L.ntaps[2]) + ", " +
                           std::to_string(L.ntaps[3]) + ">",
                       2.0 * macs,
                       bytes - (double)L.wpk_bytes + (double)L.wpk_m_bytes);
        ZJAI_HIP(launch_conv_tr_merged(L.dtype, p, ctx.stream));
        return y;
    }
    // conv3x3_m32's 256-position tiles carry twice the work of conv_igemm's 64-channel ones: with
    // 128 input channels and few tiles the smaller tiles fill the chip better. The two kernels
    // sum each output in different orders (16 channels per MFMA against 32), so the choice is
    // made from one batch item's tile count, never the batch's: a tile's 16-bit result does not
    // depend on how many tiles of its shape share its launch. 43 tiles per item is 256 workgroups
    // for the 6-tile batches of a 4K picture.
    const int tw32 = conv3x3_m32_width(OH, OW);
    const long long item_tiles32 = L.wpk32 ? (long long)((OW + tw32 - 1) / tw32) *
                                                 ((OH + 256 / tw32 - 1) / (256 / tw32)) * (L.cout / L.mt32)
                                           : 0;
    if (L.wpk32 && (L.cin == 64 || item_tiles32 >= 43) && !e.w_batch && !plane && ps == 1 && !e.relu6_in &&
        !(ctx.top().flags & ZJAI_CTX_MFMA16_CONV3X3)) {
        static const char* ty[] = {"float", "_Float16", "__bf16"};
        const int tw = tw32;
        p.w = L.wpk32;
        char name[64];
        snprintf(name, sizeof name, "conv3x3_m32<%s, %d, %d>", ty[L.dtype], L.mt32, tw);
        LaunchScope sc(ctx, name, 2.0 * macs, bytes);
        ZJAI_HIP(launch_conv3x3_m32(L.dtype, L.mt32, tw, p, ctx.stream));
        return y;
    }
    if (L.kind == CK_1x1 && !(ctx.top().flags & ZJAI_CTX_IGEMM_CONV1X1) && conv1x1_ring_ok(p, L.dtype)) {
        static const char* ty[] = {"float", "_Float16", "__bf16"};
        char name[64];
        snprintf(name, sizeof name, "conv1x1_ring<%s, %d>", ty[L.dtype], conv1x1_ring_nb(p) * 16);
        LaunchScope sc(ctx, name, 2.0 * macs, bytes);
        ZJAI_HIP(launch_conv1x1_ring(L.dtype, p, ctx.stream));
        return y;
    }
    const TileCfg cfg = launch_tile_cfg(L, N, OH, OW);
    p.ntiles = L.groups * L.nblk_g / (cfg.wc * cfg.cf);
    LaunchScope sc(ctx, conv_kernel_name(L.kind, L.dtype, cfg), 2.0 * macs, bytes);
    ZJAI_HIP(launch_conv(L.kind, L.dtype, cfg, p, ctx.stream));
    return y;
}

TensorP conv_forward(Context& ctx, const Layer& L, const TensorP& x, const Epilogue& e,
                     const TensorP& dst, const PlaneOut* plane) {
    TensorP y = conv_forward_impl(ctx, L, x, e, dst, plane);
    if (y) count_f16_range(ctx, *y);
    return y;
}

// -------------------------------------------------------------------- attention + projection
std::shared_ptr<void> attention_fold(Context& ctx, const TensorP& qkv, int heads, const float* temperature,
                                     const Layer& proj, long long* w_bstride) {
    const int dim = qkv->c / 3, c = dim / heads, N = qkv->n;
    if (proj.kind != CK_1x1 || proj.groups != 1 || proj.depthwise || proj.transposed || !proj.w_f32 ||
        proj.cin != dim || proj.cout != dim || proj.dtype != qkv->dtype)
        throw Error(ZJAI_E_INVALID_ARGUMENT, "attention: projection is not a dense dim x dim 1x1 layer");
    if (!attention_gram_fits(qkv->dtype, dim))
        throw Error(ZJAI_E_UNSUPPORTED, "attention: dim too large for the Gram kernel's LDS stage");
    const int n = qkv->h * qkv->w, nchunk = std::max(attention_gram_chunks(qkv->h, qkv->w), 1);
    const int total = heads * (c * c + 2 * c);
    const double es = dtype_size(qkv->dtype);
    float* partial = (float*)ctx.pool.alloc(sizeof(float) * N * ((size_t)nchunk * total + (size_t)dim * c));
    std::shared_ptr<void> keep(partial, [&ctx](void* q) { ctx.pool.release(q); });
    float* attn = partial + (size_t)N * nchunk * total;
    void* wfold = ctx.pool.alloc(proj.wpk_bytes * N);
    std::shared_ptr<void> out(wfold, [&ctx](void* q) { ctx.pool.release(q); });
    *w_bstride = (long long)(proj.wpk_bytes / dtype_size(proj.dtype));
    const int CK = 64 / dtype_size(proj.dtype);
    if (proj.nblk_g * 16 != dim || proj.nchunks * CK != dim)  // padded rows / columns stay zero
        ZJAI_HIP(launch_zero(wfold, proj.wpk_bytes * N, ctx.stream));
    {
        LaunchScope sc(ctx, attention_gram_name(qkv->v, qkv->dtype, dim, heads, qkv->w), 2.0 * N * total * n, es * N * 2 * dim * n + 4.0 * N * nchunk * total);
        ZJAI_HIP(launch_attention_gram(qkv->v, qkv->dtype, N, dim, heads, qkv->h, qkv->w, partial, ctx.stream));
    }
    {
        LaunchScope sc(ctx, "k_attention_softmax", 0.0, 4.0 * N * nchunk * total);
        ZJAI_HIP(launch_attention_softmax(partial, N, nchunk, dim, heads, temperature, attn, ctx.stream));
    }
    {
        LaunchScope sc(ctx, kname("k_attention_fold", proj.dtype), 2.0 * N * dim * dim * c, 4.0 * dim * dim + es * N * dim * dim);
        ZJAI_HIP(launch_attention_fold(proj.w_f32, attn, N, dim, heads, proj.dtype, proj.nblk_g, wfold,
                                       *w_bstride, ctx.stream));
    }
    return out;
}

}  // namespace zjai
