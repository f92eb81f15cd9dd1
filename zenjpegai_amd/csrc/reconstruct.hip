// Latent reconstruction of one component on the device: region geometry
// (src/tools/regions.rs:47-150) and the region-by-region driver of `reconstruct_latent`
// (src/decoder/reconstruct.rs:81-234). Host code: the hyper-decoder and the context model run
// on the conv kernels (graph.hip), the data movement on latent.hip's kernels.

#include <algorithm>
#include <map>

#include "runtime.h"

namespace zjai {

namespace {

// `axis_coords` (src/tools/regions.rs:47-71): region [start, end) along one axis at 1 / 2^depth.
std::vector<std::pair<int, int>> axis_coords(int size, int n, int depth, bool partitioned) {
    const int feature = ceil_div(size, 1 << depth);
    if (!partitioned) return {{0, feature}};
    const int region = (ceil_div(size, 128) / n) * 128;
    std::vector<std::pair<int, int>> out;
    for (int i = 0; i < n; ++i) {
        const int start = (int)(((long long)i * region) >> depth);
        const int end = i + 1 < n ? (int)(((long long)(i + 1) * region) >> depth) : feature;
        out.push_back({start, end});
    }
    return out;
}

// `grid` (src/tools/regions.rs:73-101): areas grown by `extend` towards their neighbours.
std::vector<RArea> grid(const std::vector<std::pair<int, int>>& ver, const std::vector<std::pair<int, int>>& hor,
                        int extend) {
    std::vector<RArea> out;
    for (size_t vi = 0; vi < ver.size(); ++vi)
        for (size_t hi = 0; hi < hor.size(); ++hi) {
            RArea a;
            a.x = hor[hi].first;
            a.y = ver[vi].first;
            a.w = hor[hi].second - hor[hi].first;
            a.h = ver[vi].second - ver[vi].first;
            if (hi > 0) {
                a.x -= std::min(extend, a.x);
                a.w += extend;
            }
            if (hi + 1 < hor.size()) a.w += extend;
            if (vi > 0) {
                a.y -= std::min(extend, a.y);
                a.h += extend;
            }
            if (vi + 1 < ver.size()) a.h += extend;
            out.push_back(a);
        }
    return out;
}

// `hyper_crop` (src/decoder/reconstruct.rs:67-69).
int hyper_crop(int len, int divider) { return 2 * ceil_div(len, 2 * divider) - ceil_div(len, divider); }

// Pool block released at scope exit.
struct DevBuf {
    Context& c;
    void* p;
    DevBuf(Context& ctx, size_t bytes) : c(ctx), p(ctx.pool.alloc(bytes ? bytes : 4)) {}
    ~DevBuf() { c.pool.release(p); }
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    template <typename T>
    T* as() const {
        return (T*)p;
    }
};

}  // namespace

RegionGrid region_grid(int height, int width, int ccs, const RegionParams& r, int plane) {
    if (height <= 0 || width <= 0) throw Error(ZJAI_E_INVALID_ARGUMENT, "region grid: empty picture");
    if (r.partitioned && (r.num_ver < 1 || r.num_hor < 1))
        throw Error(ZJAI_E_INVALID_ARGUMENT, "region grid: region counts must be positive");
    if (r.hyper_decoder_overlap < 0 || r.mcm_overlap < 0)
        throw Error(ZJAI_E_INVALID_ARGUMENT, "region grid: negative overlap");
    // The grid of a chroma component is built on the half-size plane scaled back up by 2.
    const int h = ccs == 0 ? height : 2 * ceil_div(height, 2);
    const int w = ccs == 0 ? width : 2 * ceil_div(width, 2);
    const int rows = r.partitioned ? r.num_ver : 1, cols = r.partitioned ? r.num_hor : 1;
    const int hd = r.hyper_decoder_overlap * 2, mcm = r.mcm_overlap * 4;
    int depth, extend;
    switch (plane) {
        case PLANE_LATENT: depth = 4; extend = mcm >> 1; break;
        case PLANE_PSI: depth = 5; extend = mcm >> 2; break;
        case PLANE_HYPER_LATENT: depth = 6; extend = hd; break;
        case PLANE_IMAGE: depth = 0; extend = 64 * hd; break;
        default: throw Error(ZJAI_E_INVALID_ARGUMENT, "region grid: unknown plane");
    }
    if (r.independent) extend = 0;
    const auto ver = axis_coords(h, rows, depth, r.partitioned);
    const auto hor = axis_coords(w, cols, depth, r.partitioned);
    RegionGrid g;
    g.rows = rows;
    g.cols = cols;
    g.core = grid(ver, hor, 0);
    g.extended = grid(ver, hor, extend);
    return g;
}

void reconstruct_latent(Context& ctx, const Net& net, int height, int width, const RegionParams& rp,
                        const int8_t* z_hat, int zh, int zw, const float* residual, int H, int W, float* psi_out,
                        float* y_out) {
    if (net.kind != NET_LATENT) throw Error(ZJAI_E_INVALID_ARGUMENT, "reconstruct_latent: not a latent model");
    if (!z_hat || !residual || !psi_out || !y_out) throw Error(ZJAI_E_INVALID_ARGUMENT, "reconstruct_latent: null buffer");
    if (zh <= 0 || zw <= 0 || H <= 0 || W <= 0) throw Error(ZJAI_E_INVALID_ARGUMENT, "reconstruct_latent: empty plane");
    const int C = net.chs, ccs = net.comp, dt = net.dtype;
    const RegionGrid img = region_grid(height, width, ccs, rp, PLANE_IMAGE);
    const RegionGrid zg = region_grid(height, width, ccs, rp, PLANE_HYPER_LATENT);
    const RegionGrid pg = region_grid(height, width, ccs, rp, PLANE_PSI);
    const RegionGrid lg = region_grid(height, width, ccs, rp, PLANE_LATENT);
    const int n = (int)img.extended.size();
    const int ph = ceil_div(H, 2), pw = ceil_div(W, 2);
    const size_t zn = (size_t)C * zh * zw, rn = (size_t)C * H * W, pn = (size_t)4 * C * ph * pw;

    DevBuf zdev(ctx, zn), rdev(ctx, rn * 4), psi(ctx, pn * 4), yhat(ctx, rn * 4);
    ZJAI_HIP(hipMemcpyAsync(zdev.p, z_hat, zn, hipMemcpyHostToDevice, ctx.stream));
    ZJAI_HIP(hipMemcpyAsync(rdev.p, residual, rn * 4, hipMemcpyHostToDevice, ctx.stream));
    ZJAI_HIP(launch_zero(psi.p, pn * 4, ctx.stream));
    ZJAI_HIP(launch_zero(yhat.p, rn * 4, ctx.stream));

    // Regions of one shape run as one batch (up to MAXB) through each network; the results are
    // merged region by region in raster order afterwards, so where extended regions overlap the
    // later one wins, as in the reference.
    auto batches = [&](auto key_of) {
        std::vector<std::vector<int>> out;
        std::map<std::vector<int>, int> slot;
        for (int r = 0; r < n; ++r) {
            const std::vector<int> k = key_of(r);
            auto it = slot.find(k);
            if (it == slot.end() || out[it->second].size() == (size_t)MAXB) {
                slot[k] = (int)out.size();
                out.push_back({});
            }
            out[slot[k]].push_back(r);
        }
        return out;
    };
    auto item = [](const TensorP& t, int b) {
        View v = t->v;
        v.p = (char*)v.p + (long long)b * v.bstride * dtype_size(t->dtype);
        return v;
    };

    // 1. psi per region (hyper-decoder on the region's z window), merged in raster order.
    std::vector<int> oh(n), ow(n);
    for (int r = 0; r < n; ++r) {
        const RArea it = img.extended[r], zt = zg.extended[r];
        const int th = ccs == 0 ? it.h : ceil_div(it.h, 2), tw = ccs == 0 ? it.w : ceil_div(it.w, 2);
        const int divider = ccs == 0 ? 32 : 16;
        oh[r] = 2 * zt.h - hyper_crop(th, divider);
        ow[r] = 2 * zt.w - hyper_crop(tw, divider);
        if (oh[r] <= 0 || ow[r] <= 0) throw Error(ZJAI_E_INVALID_ARGUMENT, "reconstruct_latent: region geometry");
        if (zt.h <= 0 || zt.w <= 0 || zt.y + zt.h > zh || zt.x + zt.w > zw)
            throw Error(ZJAI_E_INVALID_ARGUMENT, "reconstruct_latent: z_hat window outside tensor");
    }
    std::vector<TensorP> psi_of(n);
    std::vector<int> psi_item(n);
    for (const auto& bt : batches([&](int r) {
             const RArea zt = zg.extended[r];
             return std::vector<int>{zt.h, zt.w, oh[r], ow[r]};
         })) {
        ctx.check_stop();
        const int nb = (int)bt.size();
        const RArea z0 = zg.extended[bt[0]];
        Windows win{};
        for (int i = 0; i < nb; ++i) {
            win.x0[i] = zg.extended[bt[i]].x;
            win.y0[i] = zg.extended[bt[i]].y;
        }
        TensorP z = ctx.alloc(nb, C, z0.h, z0.w, dt);
        {
            LaunchScope sc(ctx, kname("k_i8_planar_to_nhwc", dt), 0.0, (1.0 + dtype_size(dt)) * nb * C * z0.h * z0.w);
            ZJAI_HIP(launch_i8_planar_to_nhwc(zdev.as<int8_t>(), C, zh, zw, win, nb, z0.h, z0.w, z->v, dt, ctx.stream));
        }
        TensorP t = hyper_decoder_forward(ctx, net, z, oh[bt[0]], ow[bt[0]]);
        for (int i = 0; i < nb; ++i) {
            psi_of[bt[i]] = t;
            psi_item[bt[i]] = i;
        }
    }
    for (int r = 0; r < n; ++r) {
        const TensorP& t = psi_of[r];
        const RArea core = pg.extended[r];
        const int h = std::max(0, std::min({core.h, t->h, ph - core.y}));
        const int w = std::max(0, std::min({core.w, t->w, pw - core.x}));
        LaunchScope sc(ctx, kname("k_assign_from_nhwc", dt), 0.0, (4.0 + dtype_size(dt)) * 4 * C * h * w);
        ZJAI_HIP(launch_assign_from_nhwc(item(t, psi_item[r]), dt, 4 * C, t->h, t->w, 0, 0, h, w, psi.as<float>(), ph,
                                         pw, core.y, core.x, ctx.stream));
    }
    psi_of.clear();

    // 2. y_hat per region (context model on the region's residual and psi windows), merged in
    // raster order: independent regions keep their whole latent area, dependent ones drop one
    // latent sample on each interior side (HD_MCM_TILE_OVERLAP / 2 / 16, reconstruct.rs:30-34).
    for (int r = 0; r < n; ++r) {
        const RArea lt = lg.extended[r], pt = pg.extended[r];
        if (lt.h <= 0 || lt.w <= 0 || lt.y + lt.h > H || lt.x + lt.w > W || pt.h <= 0 || pt.w <= 0 ||
            pt.y + pt.h > ph || pt.x + pt.w > pw)
            throw Error(ZJAI_E_INVALID_ARGUMENT, "reconstruct_latent: region window outside tensor");
    }
    std::vector<std::shared_ptr<DevBuf>> ytile_of(n);
    std::vector<int> y_item(n);
    for (const auto& bt : batches([&](int r) {
             const RArea lt = lg.extended[r], pt = pg.extended[r];
             return std::vector<int>{lt.h, lt.w, pt.h, pt.w};
         })) {
        ctx.check_stop();
        const int nb = (int)bt.size();
        const RArea l0 = lg.extended[bt[0]], p0 = pg.extended[bt[0]];
        Windows pwin{}, rwin{};
        for (int i = 0; i < nb; ++i) {
            pwin.x0[i] = pg.extended[bt[i]].x;
            pwin.y0[i] = pg.extended[bt[i]].y;
            rwin.x0[i] = lg.extended[bt[i]].x;
            rwin.y0[i] = lg.extended[bt[i]].y;
        }
        TensorP ps = ctx.alloc(nb, 4 * C, p0.h, p0.w, dt);
        {
            LaunchScope sc(ctx, kname("k_planar_to_nhwc", dt), 0.0, (4.0 + dtype_size(dt)) * nb * 4 * C * p0.h * p0.w);
            ZJAI_HIP(launch_planar_to_nhwc(psi.as<float>(), 4 * C, ph, pw, pwin, nb, p0.h, p0.w, ps->v, dt, ctx.stream));
        }
        auto ytile = std::make_shared<DevBuf>(ctx, (size_t)nb * C * l0.h * l0.w * 4);
        latent_decompress(ctx, net, rdev.as<float>(), W, (long long)H * W, rwin, l0.h, l0.w, ps, ytile->as<float>());
        for (int i = 0; i < nb; ++i) {
            ytile_of[bt[i]] = ytile;
            y_item[bt[i]] = i;
        }
    }
    for (int r = 0; r < n; ++r) {
        const RArea lt = lg.extended[r], it = img.extended[r];
        RArea core = lt;
        int ox = 0, oy = 0;
        if (!rp.independent) {
            const int cut = 48 / 2 / 16;
            const int left = it.x == 0 ? 0 : cut, top = it.y == 0 ? 0 : cut;
            const int right = it.x + it.w >= width ? 0 : cut, bottom = it.y + it.h >= height ? 0 : cut;
            if (lt.w < left + right || lt.h < top + bottom)
                throw Error(ZJAI_E_INVALID_ARGUMENT, "reconstruct_latent: region smaller than its overlap");
            core = RArea{lt.x + left, lt.y + top, lt.w - left - right, lt.h - top - bottom};
            ox = left;
            oy = top;
        }
        const int h = std::max(0, std::min({core.h, lt.h - oy, H - core.y}));
        const int w = std::max(0, std::min({core.w, lt.w - ox, W - core.x}));
        const float* src = ytile_of[r]->as<float>() + (size_t)y_item[r] * C * lt.h * lt.w;
        LaunchScope sc(ctx, "k_assign_planar", 0.0, 8.0 * C * h * w);
        ZJAI_HIP(launch_assign_planar(src, C, lt.h, lt.w, oy, ox, h, w, yhat.as<float>(), H, W, core.y, core.x,
                                      ctx.stream));
    }
    ZJAI_HIP(hipMemcpyAsync(psi_out, psi.p, pn * 4, hipMemcpyDeviceToHost, ctx.stream));
    ZJAI_HIP(hipMemcpyAsync(y_out, yhat.p, rn * 4, hipMemcpyDeviceToHost, ctx.stream));
    ZJAI_HIP(hipStreamSynchronize(ctx.stream));
}

}  // namespace zjai
