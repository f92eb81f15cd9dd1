// The synthesis transforms as fused launch sequences.
//
// Each forward restates a reference forward (src/model/synthesis.rs, src/model/attention.rs)
// with its elementwise steps folded into the conv epilogues:
//   LightResidualBlock  relu(conv(x)) + x          -> one conv, ACT_RELU + RES_ADD
//   ResidualBlock       conv2(relu(conv1(x))) + x  -> conv ACT_RELU; conv RES_ADD
//   ResAU               x * (1 + conv2(conv(relu6(x))))
//                                                  -> conv with relu6 on load; 1x1 RES_GATE
//                                                     written in place over x
//   Upsample (SOP)      pad(0,1,0,1), conv2x2, pixel_shuffle(2) -> one conv, ps = 2
//   CAB                 x + trunk * sigmoid(mask)  -> upscale convT with RES_CAB
//   crop                                           -> a view (no copy)
//   cat                                            -> producers write channel slices
//   last layer          pixel shuffle + denormalise + tile-core crop + chroma subsampling +
//                       quantisation -> the last conv's epilogue writes picture samples
//   channel attention   attn . v then project_out  -> project_out folded with attn into one
//                                                     1x1 conv over v (+ skip)

#include "runtime.h"

namespace zjai {

// ------------------------------------------------------------------------------- building
namespace {

struct Builder {
    Context& ctx;
    Net& net;
    const std::map<std::string, Param>& P;

    const Param& get(const std::string& name, std::vector<int> shape) {
        auto it = P.find(name);
        if (it == P.end()) throw Error(ZJAI_E_MODEL, name + ": missing");
        if (!shape.empty() && it->second.shape != shape) throw Error(ZJAI_E_MODEL, name + ": unexpected shape");
        if (!it->second.data) throw Error(ZJAI_E_MODEL, name + ": no data");
        return it->second;
    }
    const float* bias(const std::string& pfx, int n, bool required) {
        auto it = P.find(pfx + ".bias");
        if (it == P.end()) {
            if (required) throw Error(ZJAI_E_MODEL, pfx + ".bias: missing");
            return nullptr;
        }
        return get(pfx + ".bias", {n}).data;
    }
    // load::conv (src/model/load.rs:11-43)
    void conv(const std::string& pfx, int cin, int cout, int kh, int kw, int stride, int pad,
              int groups, bool with_bias, const int* extra = nullptr, bool keep_f32 = false) {
        const Param& w = get(pfx + ".weight", {cout, cin / groups, kh, kw});
        const float* b = with_bias ? bias(pfx, cout, true) : nullptr;
        net.L[pfx] = make_conv(ctx, cin, cout, kh, kw, stride, pad, pad, groups, w.data, b, extra,
                               net.dtype, keep_f32);
    }
    void conv3x3(const std::string& pfx, int cin, int cout, int groups, bool b) {
        conv(pfx, cin, cout, 3, 3, 1, 1, groups, b);
    }
    void conv1x1(const std::string& pfx, int cin, int cout, bool b, bool keep_f32 = false) {
        conv(pfx, cin, cout, 1, 1, 1, 0, 1, b, nullptr, keep_f32);
    }
    // load::conv_transpose (src/model/load.rs:70-89): always biased.
    void conv_t(const std::string& pfx, int cin, int cout, int k, int pad, int out_pad) {
        const Param& w = get(pfx + ".weight", {cin, cout, k, k});
        const float* b = bias(pfx, cout, true);
        net.L[pfx] = make_conv_transpose(ctx, cin, cout, k, 2, pad, out_pad, w.data, b, net.dtype);
    }
    void vec(const std::string& name, int n, std::vector<int> shape) {
        const Param& p = get(name, shape);
        float* d = nullptr;
        ZJAI_HIP(hipMalloc(&d, sizeof(float) * n));
        net.vec[name] = d;
        net.vec_bytes += sizeof(float) * n;
        ZJAI_HIP(hipMemcpy(d, p.data, sizeof(float) * n, hipMemcpyHostToDevice));
    }
    // ResAu::load (src/model/synthesis.rs:33-60): the weight's dim 1 decides the groups.
    void res_au(const std::string& pfx, int chs) {
        auto it = P.find(pfx + ".conv.weight");
        if (it == P.end() || it->second.shape.size() != 4) throw Error(ZJAI_E_MODEL, pfx + ".conv.weight: missing or malformed");
        const int per_group = it->second.shape[1];
        if (per_group <= 0 || chs % per_group) throw Error(ZJAI_E_MODEL, pfx + ".conv.weight: missing or malformed");
        conv3x3(pfx + ".conv", chs, chs, chs / per_group, false);
        conv1x1(pfx + ".conv2", chs, chs, false);
    }
    void res_block(const std::string& pfx, int c) {
        conv3x3(pfx + ".conv1", c, c, 1, true);
        conv3x3(pfx + ".conv2", c, c, 1, true);
    }
    void upsample(int op, const std::string& pfx, int cin, int cout) {
        if (op == OP_BOP) {
            conv_t(pfx, cin, cout, 4, 1, 0);
        } else {
            static const int extra[4] = {0, 0, 1, 1};  // F.pad(x, (0, 1, 0, 1))
            conv(pfx + ".conv", cin, cout * 4, 2, 2, 1, 0, 1, false, extra);
        }
    }
    void cab(const std::string& pfx, int c) {
        res_block(pfx + ".residual_trunk.0", c);
        res_block(pfx + ".residual_trunk.1", c);
        conv(pfx + ".subscale", c, c, 3, 3, 2, 1, 1, true);
        res_block(pfx + ".residual_mask2.0", c);
        res_block(pfx + ".residual_mask3.0", c);
        conv_t(pfx + ".upscale", c, c, 3, 1, 1);
    }
    void transformer_block(const std::string& p, int dim) {
        const int hidden = dim * 4;
        vec(p + ".prep_data.norm1.weight", dim, {dim});
        vec(p + ".prep_data.norm1.bias", dim, {dim});
        conv1x1(p + ".prep_data.conv1", dim, 3 * dim, false);
        conv(p + ".prep_data.conv2", 3 * dim, 3 * dim, 3, 3, 1, 1, 3 * dim, false);
        vec(p + ".attn.temperature", 4, {4, 1, 1});
        conv1x1(p + ".attn.project_out", dim, dim, false, true);
        vec(p + ".ffn.norm1.weight", dim, {dim});
        vec(p + ".ffn.norm1.bias", dim, {dim});
        conv1x1(p + ".ffn.project_in", dim, 2 * hidden, false);
        conv(p + ".ffn.dwconv", 2 * hidden, 2 * hidden, 3, 3, 1, 1, 2 * hidden, false);
        conv1x1(p + ".ffn.project_out", hidden, dim, false);
    }
    // A 3x3 stride-2 conv over picture planes: input channels padded to a multiple of 8 with
    // zero weights (the kernels read whole 16-byte channel vectors; the padded input channels
    // are zeros too, so the extra products are exact zeros).
    void conv_s2_planes(const std::string& pfx, int cin, int cout) {
        const Param& w = get(pfx + ".weight", {cout, cin, 3, 3});
        const float* b = bias(pfx, cout, true);
        const int cp = round_up(cin, 8);
        std::vector<float> wp((size_t)cout * cp * 9, 0.0f);
        for (int o = 0; o < cout; ++o)
            for (int i = 0; i < cin; ++i)
                for (int k = 0; k < 9; ++k) wp[((size_t)o * cp + i) * 9 + k] = w.data[((size_t)o * cin + i) * 9 + k];
        net.L[pfx] = make_conv(ctx, cp, cout, 3, 3, 2, 1, 1, 1, wp.data(), b, nullptr, net.dtype, false);
    }
    // `clip_bounds` (src/model/load.rs:94-101): optional [lo, hi] lists; the first n channels
    // (the shorter list, at most the map's channels) are clipped.
    void clip_bounds(const std::string& key, int stage, int chs) {
        auto lo = P.find(key + ".MinList"), hi = P.find(key + ".MaxList");
        if (lo == P.end() || hi == P.end()) return;
        auto numel = [](const Param& q) {
            long long n = 1;
            for (int d : q.shape) n *= d;
            return n;
        };
        const int n = (int)std::min<long long>({numel(lo->second), numel(hi->second), (long long)chs});
        if (n <= 0) return;
        if (!lo->second.data || !hi->second.data) throw Error(ZJAI_E_MODEL, key + ": no data");
        for (auto* q : {&lo, &hi}) {
            float* d = nullptr;
            ZJAI_HIP(hipMalloc(&d, sizeof(float) * n));
            net.vec[(*q)->first] = d;
            net.vec_bytes += sizeof(float) * n;
            ZJAI_HIP(hipMemcpy(d, (*q)->second.data, sizeof(float) * n, hipMemcpyHostToDevice));
        }
        net.clip_n[stage] = n;
    }
    void tam(const std::string& pfx, int dim, bool ds) {
        if (ds) {
            conv(pfx + ".ds_conv", dim, dim, 3, 3, 2, 1, 1, true);
            conv_t(pfx + ".us_conv", dim, dim, 3, 1, 1);
        }
        transformer_block(pfx + ".TABs.0", dim);
        transformer_block(pfx + ".TABs.1", dim);
    }
};

}  // namespace

Net::~Net() {
    for (auto& kv : vec) (void)hipFree(kv.second);
}

NetP build_net(Context& ctx, int op, int comp, int dtype, const std::map<std::string, Param>& params) {
    if (op < OP_SOP || op > OP_HOP || comp < COMP_Y || comp > COMP_UV)
        throw Error(ZJAI_E_INVALID_ARGUMENT, "net: unknown operating point / component");
    auto net = std::make_shared<Net>();
    net->op = op;
    net->comp = comp;
    net->dtype = dtype;
    Builder b{ctx, *net, params};
    if (comp == COMP_Y && op != OP_HOP) {
        // LightPrimary::load (src/model/synthesis.rs:526-548)
        const int c1 = 64, c2 = op == OP_SOP ? 32 : 64, c3 = op == OP_SOP ? 32 : 96;
        b.conv3x3("first_stage.0.0.conv1", 160, 160, 1, true);
        b.upsample(op, "first_stage.1", 160, c1);
        b.res_au("first_stage.2", c1);
        b.upsample(op, "conv2_t", c1, c2);
        b.res_au("iact2", c2);
        b.conv3x3("conv3", c2, c3, 1, true);
        b.res_au("iact3", c3);
        b.conv1x1("conv4", c3, 16, false);
    } else if (comp == COMP_Y) {
        // HopPrimary::load (src/model/synthesis.rs:339-354)
        const int c = 128;
        b.res_block("first_stage.0.0", 160);
        b.conv_t("first_stage.1", 160, c, 3, 1, 1);
        b.res_au("first_stage.2", c);
        b.conv_t("conv2_t", c, c, 3, 1, 1);
        b.cab("CAB", c);
        b.res_au("iact2", c);
        b.conv1x1("conv3_t", c, 4 * c, true);
        b.tam("TAM", c, true);
        b.res_au("iact3", c);
        b.conv_t("conv4_t", c, 1, 3, 1, 1);
    } else {
        // SynthesisSecondary::load (src/model/synthesis.rs:972-990)
        b.conv3x3("first_stage.conv1", 256, 48, 1, true);
        if (op == OP_HOP) {
            const int c = 64;  // HopSecondary::load (:740-753)
            b.conv_t("conv2_t", 144, c, 3, 1, 1);
            b.cab("CAB", c);
            b.res_au("iact2", c);
            b.conv1x1("conv3_t", c, 4 * c, true);
            b.tam("TAM", c, false);
            b.res_au("iact3", c);
            b.conv_t("conv4_t", c, 8, 3, 1, 1);
        } else {
            // LightSecondary::load (:871-888)
            const int c2 = op == OP_SOP ? 32 : 64, c3 = op == OP_SOP ? 32 : 128;
            b.upsample(op, "conv2_t", 144, c2);
            b.res_au("iact2", c2);
            b.conv3x3("conv3", c2, c3, 1, true);
            b.res_au("iact3", c3);
            b.conv1x1("conv4", c3, 128, false);
        }
    }
    return net;
}

NetP build_latent_net(Context& ctx, int comp, int dtype, const std::map<std::string, Param>& params) {
    if (comp < COMP_Y || comp > COMP_UV) throw Error(ZJAI_E_INVALID_ARGUMENT, "latent model: unknown component");
    auto net = std::make_shared<Net>();
    net->kind = NET_LATENT;
    net->comp = comp;
    net->dtype = dtype;
    const int c = comp == COMP_Y ? 160 : 96;  // LATENT_CHANNELS (src/header.rs:31)
    net->chs = c;
    Builder b{ctx, *net, params};
    // HyperDecoder::load (src/model/hyper_decoder.rs:24-45)
    b.conv1x1("hyper_decoder.conv1", c, c, false);
    b.conv_t("hyper_decoder.conv2", c, c, 4, 1, 0);
    b.conv3x3("hyper_decoder.conv3", c, c, 1, true);
    b.conv3x3("hyper_decoder.conv4", c, 4 * c, 1, true);
    // ContextModel::load (src/model/mcm.rs:123-159), when the checkpoint has one
    // (src/model/common.rs:117-121).
    if (params.count("context.MCM.0.fusion_pred_net.conv1.weight")) {
        net->context = true;
        for (int s = 0; s < 4; ++s) {
            const std::string p = "context.MCM." + std::to_string(s);
            if (s > 0) {
                b.conv1x1(p + ".conv.0", s * c, c, false);
                b.conv3x3(p + ".conv.1", c, c, c / 32, true);
            }
            b.conv1x1(p + ".fusion_pred_net.conv1", s == 0 ? c : 2 * c, c, false);
            b.conv1x1(p + ".fusion_pred_net.conv2", c, c, false);
            b.conv1x1(p + ".fusion_pred_net.conv3", c, c, false);
        }
    }
    return net;
}

NetP build_analysis_net(Context& ctx, int op, int comp, int dtype, const std::map<std::string, Param>& params) {
    if (comp < COMP_Y || comp > COMP_UV) throw Error(ZJAI_E_INVALID_ARGUMENT, "analysis transform: unknown component");
    // check_op (src/model/analysis.rs:209-217)
    if (op == OP_SOP) throw Error(ZJAI_E_INVALID_ARGUMENT, "there is no SOP analysis transform (use BOP)");
    if (op != OP_BOP && op != OP_HOP) throw Error(ZJAI_E_INVALID_ARGUMENT, "analysis transform: unknown operating point");
    auto net = std::make_shared<Net>();
    net->kind = NET_ANALYSIS;
    net->op = op;
    net->comp = comp;
    net->dtype = dtype;
    net->chs = comp == COMP_Y ? 160 : 96;  // LATENT_CHANNELS (src/header.rs:31)
    net->in_ch = comp == COMP_Y ? 1 : 12;
    const int C = 128;  // hidden width (src/model/analysis.rs:32)
    const bool hop = op == OP_HOP;
    Builder b{ctx, *net, params};
    // Trunk::load (src/model/analysis.rs:122-153)
    b.conv_s2_planes("conv1", net->in_ch, C);
    b.res_au("act1", C);
    if (hop) b.tam("TAM", C, comp == COMP_Y);
    b.conv("conv2", C, C, 3, 3, 2, 1, 1, true);
    b.res_au("act2", C);
    if (hop) b.cab("cab", C);
    b.conv("conv3", C, C, 3, 3, 2, 1, 1, true);
    b.res_au("act3", C);
    if (comp == COMP_Y) {
        b.conv("conv4", C, net->chs, 3, 3, 2, 1, 1, true);
        b.conv1x1("conv5", net->chs, net->chs, false);
    } else {
        b.conv1x1("conv5", C, net->chs, false);
    }
    // clip_key (src/model/analysis.rs:111-119): clip_thres.E{stage}{B|H}
    for (int k = 1; k <= 5; ++k) {
        if (k == 4 && comp != COMP_Y) continue;
        const int chs = k <= 3 ? C : net->chs;
        b.clip_bounds("clip_thres.E" + std::to_string(k) + (hop ? "H" : "B"), k, chs);
    }
    return net;
}

// -------------------------------------------------------------------------------- forward
namespace {

struct Fwd {
    Context& ctx;
    const Net& net;

    const Layer& L(const std::string& name) const {
        auto it = net.L.find(name);
        if (it == net.L.end()) throw Error(ZJAI_E_MODEL, name + ": layer missing");
        return *it->second;
    }
    TensorP conv(const std::string& name, const TensorP& x, Epilogue e = Epilogue{},
                 const TensorP& dst = nullptr, const PlaneOut* plane = nullptr) {
        return conv_forward(ctx, L(name), x, e, dst, plane);
    }
    // ResAu::forward (src/model/synthesis.rs:62-74); the gate overwrites x.
    // The fused ResAU kernel applies to 32- / 64-channel ResAUs with 16-channel groups whose
    // layers are packed as one K chunk and one 16-row block per group (the 3x3) and 16-row blocks
    // (the 1x1), on a 16-byte-aligned input view.
    bool res_au_fusable(const std::string& pfx, const TensorP& x) {
        if (ctx.top().flags & ZJAI_CTX_UNFUSED_BLOCKS) return false;
        const Layer& c1 = L(pfx + ".conv");
        const Layer& c2 = L(pfx + ".conv2");
        const int C = x->c;
        if (!resau_fused_supported(C, c1.groups) || c1.kind != CK_3x3 || c1.cin != C || c1.cout != C ||
            c1.depthwise || c1.nchunks != 1 || c1.nblk_g != 1 || c1.dtype != x->dtype || c1.extra[0] ||
            c1.extra[1] || c1.extra[2] || c1.extra[3] || c1.pad_h != 1 || c1.pad_w != 1)
            return false;
        if (c2.kind != CK_1x1 || c2.groups != 1 || c2.cin != C || c2.cout != C || c2.nblk_g * 16 != C ||
            c2.dtype != x->dtype || c2.bias)
            return false;
        const View& v = x->v;
        return v.cs % 8 == 0 && v.c_off % 8 == 0 && v.row % 8 == 0 && v.bstride % 8 == 0;
    }
    TensorP res_au(const std::string& pfx, const TensorP& x) {
        if (res_au_fusable(pfx, x)) {
            const Layer& c1 = L(pfx + ".conv");
            const Layer& c2 = L(pfx + ".conv2");
            TensorP y = ctx.alloc(x->n, x->c, x->h, x->w, x->dtype);
            ResauArgs a{};
            a.x = x->v;
            a.y = y->v;
            a.N = x->n;
            a.h = x->h;
            a.w = x->w;
            a.w1 = c1.wpk;
            a.w2 = c2.wpk;
            a.nblk2 = c2.nblk_g;
            const double npos = (double)x->n * x->h * x->w, C = x->c;
            {
                char name[48];
                static const char* ty[] = {"float", "_Float16", "__bf16"};
                snprintf(name, sizeof name, "k_resau<%s, %d, %d>", ty[x->dtype], x->c, resau_rows(x->dtype, x->n, x->h, x->w));
                LaunchScope sc(ctx, name, 2.0 * npos * (C * 16 * 9 + C * C), 2.0 * dtype_size(x->dtype) * npos * C);
                ZJAI_HIP(launch_resau(x->dtype, x->c, a, ctx.stream));
            }
            count_f16_range(ctx, *y);
            return y;
        }
        Epilogue e1;
        e1.relu6_in = 1;
        TensorP t = conv(pfx + ".conv", x, e1);
        Epilogue e2;
        e2.res = RES_GATE;
        e2.r1 = x.get();
        conv(pfx + ".conv2", t, e2, x);
        return x;
    }
    // ResidualBlock::forward (src/model/attention.rs:35-43)
    TensorP res_block(const std::string& pfx, const TensorP& x) {
        Epilogue e1;
        e1.act = ACT_RELU;
        TensorP t = conv(pfx + ".conv1", x, e1);
        Epilogue e2;
        e2.res = RES_ADD;
        e2.r1 = x.get();
        return conv(pfx + ".conv2", t, e2);
    }
    // Upsample::forward (src/model/synthesis.rs:158-166)
    TensorP upsample(const std::string& pfx, const TensorP& x) {
        if (net.op == OP_BOP) return conv(pfx, x);
        Epilogue e;
        e.ps = 2;
        return conv(pfx + ".conv", x, e);
    }
    // Cab::forward (src/model/attention.rs:119-139)
    TensorP cab(const std::string& pfx, const TensorP& x) {
        TensorP trunk = res_block(pfx + ".residual_trunk.0", x);
        trunk = res_block(pfx + ".residual_trunk.1", trunk);
        TensorP m = conv(pfx + ".subscale", x);
        m = res_block(pfx + ".residual_mask2.0", m);
        m = res_block(pfx + ".residual_mask3.0", m);
        int oh, ow;
        L(pfx + ".upscale").out_size(m->h, m->w, &oh, &ow);
        if (oh != trunk->h || ow != trunk->w) throw Error(ZJAI_E_INVALID_ARGUMENT, "CAB: odd feature map size");
        Epilogue e;
        e.res = RES_CAB;
        e.r1 = trunk.get();
        e.r2 = x.get();
        return conv(pfx + ".upscale", m, e);
    }
    TensorP layer_norm(const std::string& pfx, const TensorP& x) {
        TensorP y = ctx.alloc(x->n, x->c, x->h, x->w, x->dtype);
        {
            LaunchScope sc(ctx, kname("k_layer_norm", x->dtype), 0.0, 2.0 * dtype_size(x->dtype) * x->n * x->c * x->h * x->w);
            ZJAI_HIP(launch_layer_norm(x->v, y->v, x->dtype, x->n, x->c, x->h, x->w, net.vec.at(pfx + ".weight"),
                                       net.vec.at(pfx + ".bias"), ctx.stream));
        }
        count_f16_range(ctx, *y);
        return y;
    }
    // Profile name of a fused block kernel, as the kernel symbol reads: k_ffn<__bf16, 128>,
    // k_ffn_f32<128>.
    static std::string fused_name(const char* base, int dtype, int dim) {
        if (dtype == DT_F32) return std::string(base) + "_f32<" + std::to_string(dim) + ">";
        const std::string kn = kname(base, dtype);
        return kn.substr(0, kn.size() - 1) + ", " + std::to_string(dim) + ">";
    }
    // The fused feed-forward kernel applies to nets with dim 64 / 128 whose 1x1 weights are
    // packed unpadded (K chunks of 64 bytes of channels, 16-row blocks) and whose input is a
    // whole 16-byte-aligned NHWC tensor.
    bool ffn_fusable(const std::string& p, const TensorP& x) {
        if (ctx.top().flags & ZJAI_CTX_UNFUSED_BLOCKS) return false;
        const int dim = x->c, hidden = 4 * dim;
        if (!ffn_fused_supported(x->dtype, dim)) return false;
        const Layer& pin = L(p + ".ffn.project_in");
        const Layer& dwl = L(p + ".ffn.dwconv");
        const Layer& pout = L(p + ".ffn.project_out");
        const int ck = 64 / dtype_size(x->dtype);
        if (pin.kind != CK_1x1 || pin.groups != 1 || pin.transposed || pin.dtype != x->dtype ||
            pin.nblk_g * 16 != 2 * hidden || pin.nchunks * ck != dim || pin.cin != dim)
            return false;
        if (pout.kind != CK_1x1 || pout.groups != 1 || pout.transposed || pout.dtype != x->dtype ||
            pout.nblk_g * 16 != dim || pout.nchunks * ck != hidden || pout.cin != hidden)
            return false;
        if (!dwl.depthwise || dwl.cin != 2 * hidden || !dwl.dw_w) return false;
        const View& v = x->v;
        return v.cs % 8 == 0 && v.c_off % 8 == 0 && v.row % 8 == 0 && v.bstride % 8 == 0;
    }
    // The fused prep_data kernel: same conditions, a dim -> 3 dim unpadded 1x1 and a 3 dim
    // depthwise.
    bool qkv_fusable(const std::string& p, const TensorP& x) {
        if (ctx.top().flags & ZJAI_CTX_UNFUSED_BLOCKS) return false;
        const int dim = x->c;
        if (!qkv_fused_supported(x->dtype, dim)) return false;
        const Layer& c1 = L(p + ".prep_data.conv1");
        const Layer& c2 = L(p + ".prep_data.conv2");
        const int ck = 64 / dtype_size(x->dtype);
        if (c1.kind != CK_1x1 || c1.groups != 1 || c1.transposed || c1.dtype != x->dtype ||
            c1.nblk_g * 16 != 3 * dim || c1.nchunks * ck != dim || c1.cin != dim)
            return false;
        if (!c2.depthwise || c2.cin != 3 * dim || !c2.dw_w) return false;
        const View& v = x->v;
        return v.cs % 8 == 0 && v.c_off % 8 == 0 && v.row % 8 == 0 && v.bstride % 8 == 0;
    }
    // TransformerBlock::forward (src/model/attention.rs:328-372)
    TensorP transformer_block(const std::string& p, TensorP x) {
        const int dim = x->c, heads = 4, hidden = 4 * dim;
        TensorP t;
        if (qkv_fusable(p, x)) {
            const Layer& c1 = L(p + ".prep_data.conv1");
            const Layer& c2 = L(p + ".prep_data.conv2");
            t = ctx.alloc(x->n, 3 * dim, x->h, x->w, x->dtype);
            QkvArgs a{};
            a.x = x->v;
            a.y = t->v;
            a.N = x->n;
            a.h = x->h;
            a.w = x->w;
            a.ln_w = net.vec.at(p + ".prep_data.norm1.weight");
            a.ln_b = net.vec.at(p + ".prep_data.norm1.bias");
            a.w1 = c1.wpk;
            a.nblk1 = c1.nblk_g;
            a.b1 = c1.bias;
            a.dw_w = c2.dw_w;
            a.dw_b = c2.bias;
            const double npos = (double)x->n * x->h * x->w;
            {
                LaunchScope sc(ctx, fused_name("k_qkv", x->dtype, dim),
                               2.0 * npos * (3.0 * dim * dim + 9.0 * 3 * dim),
                               (double)dtype_size(x->dtype) * npos * 4 * dim);
                ZJAI_HIP(launch_qkv_fused(a, x->dtype, dim, ctx.stream));
            }
            count_f16_range(ctx, *t);
        } else {
            t = layer_norm(p + ".prep_data.norm1", x);
            t = conv(p + ".prep_data.conv1", t);
            t = conv(p + ".prep_data.conv2", t);  // depthwise 3x3
        }
        // channel_attention + project_out: fold attn into the projection, run it on v.
        Epilogue ea;
        std::shared_ptr<void> wfold =
            attention_fold(ctx, t, heads, net.vec.at(p + ".attn.temperature"), L(p + ".attn.project_out"),
                           &ea.w_bstride);
        ea.w_batch = wfold.get();
        ea.res = RES_ADD;
        ea.r1 = x.get();
        conv(p + ".attn.project_out", channel_view(t, 2 * dim, dim), ea, x);
        t.reset();
        // x = x + ffn(x)
        if (ffn_fusable(p, x)) {
            const Layer& pin = L(p + ".ffn.project_in");
            const Layer& dwl = L(p + ".ffn.dwconv");
            const Layer& pout = L(p + ".ffn.project_out");
            TensorP y = ctx.alloc(x->n, dim, x->h, x->w, x->dtype);
            FfnArgs a{};
            a.x = x->v;
            a.y = y->v;
            a.N = x->n;
            a.h = x->h;
            a.w = x->w;
            a.ln_w = net.vec.at(p + ".ffn.norm1.weight");
            a.ln_b = net.vec.at(p + ".ffn.norm1.bias");
            a.w_in = pin.wpk;
            a.nblk_in = pin.nblk_g;
            a.b_in = pin.bias;
            a.dw_w = dwl.dw_w;
            a.dw_b = dwl.bias;
            a.w_out = pout.wpk;
            a.nblk_out = pout.nblk_g;
            a.b_out = pout.bias;
            const double npos = (double)x->n * x->h * x->w;
            {
                LaunchScope sc(ctx, fused_name("k_ffn", x->dtype, dim),
                               2.0 * npos * (2.0 * hidden * dim + 9.0 * 2 * hidden + (double)hidden * dim),
                               2.0 * dtype_size(x->dtype) * npos * dim);
                ZJAI_HIP(launch_ffn_fused(a, x->dtype, dim, ctx.stream));
            }
            count_f16_range(ctx, *y);
            return y;
        }
        TensorP u = layer_norm(p + ".ffn.norm1", x);
        u = conv(p + ".ffn.project_in", u);
        const Layer& dw = L(p + ".ffn.dwconv");
        TensorP f = ctx.alloc(u->n, hidden, u->h, u->w, u->dtype);
        {
            LaunchScope sc(ctx, kname("k_depthwise3x3", u->dtype), 2.0 * 9 * 2 * hidden * u->n * u->h * u->w,
                           (double)dtype_size(u->dtype) * 3 * hidden * u->n * u->h * u->w);
            ZJAI_HIP(launch_depthwise3x3(u->v, f->v, u->dtype, u->n, 2 * hidden, u->h, u->w, dw.dw_w, dw.bias,
                                         hidden, ctx.stream));
        }
        count_f16_range(ctx, *f);
        u.reset();
        Epilogue ef;
        ef.res = RES_ADD;
        ef.r1 = x.get();
        conv(p + ".ffn.project_out", f, ef, x);
        return x;
    }
    // Tam::forward (src/model/attention.rs:528-545)
    TensorP tam(const std::string& pfx, TensorP x, bool ds) {
        if (ds) x = conv(pfx + ".ds_conv", x);
        x = transformer_block(pfx + ".TABs.0", x);
        x = transformer_block(pfx + ".TABs.1", x);
        if (ds) x = conv(pfx + ".us_conv", x);
        return x;
    }
};

}  // namespace

void primary_out_size(int op, int h, int w, int* oh, int* ow) {
    if (op == OP_HOP) {
        *oh = 2 * ceil_div(h, 2);
        *ow = 2 * ceil_div(w, 2);
    } else {
        *oh = 4 * ceil_div(h, 4);
        *ow = 4 * ceil_div(w, 4);
    }
}

void secondary_out_size(int op, int h, int w, int* oh, int* ow) {
    if (op == OP_HOP) {
        *oh = 4 * ceil_div(h, 4);
        *ow = 4 * ceil_div(w, 4);
    } else {
        *oh = 8 * ceil_div(h, 8);
        *ow = 8 * ceil_div(w, 8);
    }
}

void primary_forward(Context& ctx, const Net& net, const TensorP& y_hat, int h, int w, const PlaneOut& out) {
    if (net.comp != COMP_Y) throw Error(ZJAI_E_INVALID_ARGUMENT, "primary forward on a chroma net");
    if (y_hat->c != 160) throw Error(ZJAI_E_INVALID_ARGUMENT, "primary: latent must have 160 channels");
    Fwd f{ctx, net};
    const int h8 = ceil_div(h, 8), w8 = ceil_div(w, 8), h4 = ceil_div(h, 4), w4 = ceil_div(w, 4);
    if (net.op != OP_HOP) {
        // LightPrimary::forward (src/model/synthesis.rs:550-580)
        Epilogue e0;
        e0.act = ACT_RELU;
        e0.res = RES_ADD;
        e0.r1 = y_hat.get();
        TensorP x = f.conv("first_stage.0.0.conv1", y_hat, e0);
        ctx.check_stop();
        x = f.upsample("first_stage.1", x);
        x = f.res_au("first_stage.2", x);
        x = crop_view(x, h8, w8);
        ctx.check_stop();
        x = f.upsample("conv2_t", x);
        x = crop_view(x, h4, w4);
        ctx.check_stop();
        x = f.res_au("iact2", x);
        ctx.check_stop();
        x = f.conv("conv3", x);
        ctx.check_stop();
        x = f.res_au("iact3", x);
        ctx.check_stop();
        Epilogue e;
        e.ps = 4;
        f.conv("conv4", x, e, nullptr, &out);
        return;
    }
    // HopPrimary::forward (src/model/synthesis.rs:356-390)
    TensorP x = f.res_block("first_stage.0.0", y_hat);
    ctx.check_stop();
    x = f.conv("first_stage.1", x);
    x = f.res_au("first_stage.2", x);
    x = crop_view(x, h8, w8);
    ctx.check_stop();
    x = f.conv("conv2_t", x);
    x = f.cab("CAB", x);
    x = crop_view(x, h4, w4);
    ctx.check_stop();
    x = f.res_au("iact2", x);
    ctx.check_stop();
    Epilogue e3;
    e3.ps = 2;
    x = f.conv("conv3_t", x, e3);
    ctx.check_stop();
    x = f.tam("TAM", x, true);
    x = crop_view(x, ceil_div(h, 2), ceil_div(w, 2));
    ctx.check_stop();
    x = f.res_au("iact3", x);
    ctx.check_stop();
    f.conv("conv4_t", x, Epilogue{}, nullptr, &out);
}

void secondary_forward(Context& ctx, const Net& net, const TensorP& y_luma, const TensorP& y_chroma,
                       int h, int w, const PlaneOut& out) {
    if (net.comp != COMP_UV) throw Error(ZJAI_E_INVALID_ARGUMENT, "secondary forward on a luma net");
    if (y_luma->c != 160 || y_chroma->c != 96)
        throw Error(ZJAI_E_INVALID_ARGUMENT, "secondary: latents must have 160 / 96 channels");
    if (y_luma->dtype != net.dtype || y_chroma->dtype != net.dtype)
        throw Error(ZJAI_E_INVALID_ARGUMENT, "secondary: latent precision differs from the net");
    // SynthesisSecondary::forward_with (src/model/synthesis.rs:1004-1038)
    const int lh = std::min(y_luma->h, y_chroma->h), lw = std::min(y_luma->w, y_chroma->w);
    if (y_chroma->h != lh || y_chroma->w != lw)
        throw Error(ZJAI_E_INVALID_ARGUMENT, "chroma latent larger than the luma latent");
    if (y_luma->n != y_chroma->n) throw Error(ZJAI_E_INVALID_ARGUMENT, "secondary: latent batch sizes differ");
    Fwd f{ctx, net};
    const int dt = net.dtype, N = y_luma->n;
    const double es = dtype_size(dt);
    // cat(luma, chroma): when the two latents already are channels 0..159 and 160..255 of one
    // 256-channel block of this shape (as zjai_picture_run lays them out), that block is the
    // concatenation and nothing is copied.
    const bool joined = y_luma->base == y_chroma->base && y_luma->v.p == y_chroma->v.p &&
                        y_luma->v.c_off == 0 && y_chroma->v.c_off == 160 && y_luma->v.cs == 256 &&
                        y_chroma->v.cs == 256 && y_luma->v.row == y_chroma->v.row &&
                        y_luma->v.bstride == y_chroma->v.bstride && y_luma->h == lh && y_luma->w == lw;
    TensorP cat;
    if (joined) {
        cat = std::make_shared<Tensor>(*y_luma);
        cat->c = 256;
    } else {
        cat = ctx.alloc(N, 256, lh, lw, dt);
        {
            LaunchScope sc(ctx, kname("k_copy", dt), 0.0, 2.0 * es * N * 160 * lh * lw);
            ZJAI_HIP(launch_copy(y_luma->v, cat->v, dt, N, 160, lh, lw, ctx.stream));
        }
        {
            LaunchScope sc(ctx, kname("k_copy", dt), 0.0, 2.0 * es * N * 96 * lh * lw);
            ZJAI_HIP(launch_copy(y_chroma->v, channel_view(cat, 160, 96)->v, dt, N, 96, lh, lw, ctx.stream));
        }
    }
    TensorP x = ctx.alloc(N, 144, lh, lw, dt);
    f.conv("first_stage.conv1", cat, Epilogue{}, channel_view(x, 0, 48));
    {
        LaunchScope sc(ctx, kname("k_copy", dt), 0.0, 2.0 * es * N * 96 * lh * lw);
        ZJAI_HIP(launch_copy(y_chroma->v, channel_view(x, 48, 96)->v, dt, N, 96, lh, lw, ctx.stream));
    }
    cat.reset();
    ctx.check_stop();
    const int h8 = ceil_div(h, 8), w8 = ceil_div(w, 8);
    if (net.op == OP_HOP) {
        // HopSecondary::forward (:755-773)
        x = f.conv("conv2_t", x);
        x = f.cab("CAB", x);
        x = crop_view(x, h8, w8);
        ctx.check_stop();
        x = f.res_au("iact2", x);
        ctx.check_stop();
        Epilogue e3;
        e3.ps = 2;
        x = f.conv("conv3_t", x, e3);
        ctx.check_stop();
        x = f.tam("TAM", x, false);
        x = crop_view(x, ceil_div(h, 4), ceil_div(w, 4));
        ctx.check_stop();
        x = f.res_au("iact3", x);
        ctx.check_stop();
        Epilogue e4;
        e4.ps = 2;
        f.conv("conv4_t", x, e4, nullptr, &out);
        return;
    }
    // LightSecondary::forward (:890-909)
    x = f.upsample("conv2_t", x);
    x = crop_view(x, h8, w8);
    ctx.check_stop();
    x = f.res_au("iact2", x);
    ctx.check_stop();
    x = f.conv("conv3", x);
    ctx.check_stop();
    x = f.res_au("iact3", x);
    ctx.check_stop();
    Epilogue e;
    e.ps = 8;
    f.conv("conv4", x, e, nullptr, &out);
}

TensorP hyper_decoder_forward(Context& ctx, const Net& net, const TensorP& z, int out_h, int out_w) {
    if (net.kind != NET_LATENT) throw Error(ZJAI_E_INVALID_ARGUMENT, "hyper-decoder: not a latent model");
    if (z->c != net.chs || z->dtype != net.dtype)
        throw Error(ZJAI_E_INVALID_ARGUMENT, "hyper-decoder: z_hat channels / precision differ from the model");
    Fwd f{ctx, net};
    TensorP x = f.conv("hyper_decoder.conv1", z);
    ctx.check_stop();
    x = f.conv("hyper_decoder.conv2", x);
    if (x->h != out_h || x->w != out_w) {
        if (out_h <= 0 || out_w <= 0 || out_h > x->h || out_w > x->w)
            throw Error(ZJAI_E_INVALID_ARGUMENT, "hyper-decoder: crop larger than the upsampled map");
        x = crop_view(x, out_h, out_w);
    }
    ctx.check_stop();
    // relu6 after the crop and after conv3 run as relu6 on the next conv's loads.
    Epilogue e;
    e.relu6_in = 1;
    x = f.conv("hyper_decoder.conv3", x, e);
    ctx.check_stop();
    return f.conv("hyper_decoder.conv4", x, e);
}

TensorP analysis_forward(Context& ctx, const Net& net, const float* x, int h, int w, bool clip) {
    if (net.kind != NET_ANALYSIS) throw Error(ZJAI_E_INVALID_ARGUMENT, "not an analysis transform");
    if (h <= 0 || w <= 0) throw Error(ZJAI_E_INVALID_ARGUMENT, "analysis transform: empty picture");
    const int dt = net.dtype;
    const double es = dtype_size(dt);
    Fwd f{ctx, net};
    // pad_amount (src/model/analysis.rs:43-46): one row / column when the map is odd.
    auto pad_amount = [](int len, int d) { return 2 * ceil_div(len, 2 * d) - ceil_div(len, d); };
    // pad_for (src/model/analysis.rs:72-81)
    auto pad_for = [&](const TensorP& t, int d) -> TensorP {
        if (t->h != ceil_div(h, d) || t->w != ceil_div(w, d))
            throw Error(ZJAI_E_INVALID_ARGUMENT, "analysis transform: map size does not match the picture size");
        const int ph = pad_amount(h, d), pw = pad_amount(w, d);
        if (!ph && !pw) return t;
        TensorP o = ctx.alloc(t->n, t->c, t->h + ph, t->w + pw, dt);
        LaunchScope sc(ctx, kname("k_replicate_pad", dt), 0.0, 2.0 * es * o->n * o->c * o->h * o->w);
        ZJAI_HIP(launch_replicate_pad(t->v, dt, t->n, t->c, t->h, t->w, o->v, o->h, o->w, ctx.stream));
        return o;
    };
    // feature clipping after conv k (src/model/analysis.rs:169-203, :258-266)
    auto clip_after = [&](const TensorP& t, int k) {
        if (!clip || !net.clip_n[k]) return;
        const std::string key = std::string("clip_thres.E") + std::to_string(k) + (net.op == OP_HOP ? "H" : "B");
        LaunchScope sc(ctx, kname("k_clip_channels", dt), 0.0, 2.0 * es * t->n * net.clip_n[k] * t->h * t->w);
        ZJAI_HIP(launch_clip_channels(t->v, dt, t->n, t->c, t->h, t->w, net.clip_n[k], net.vec.at(key + ".MinList"),
                                      net.vec.at(key + ".MaxList"), ctx.stream));
    };
    // normalize + the first padding_layer, channels padded to the first conv's input width
    const int cp = round_up(net.in_ch, 8);
    TensorP in = ctx.alloc(1, cp, h + pad_amount(h, 1), w + pad_amount(w, 1), dt);
    {
        LaunchScope sc(ctx, kname("k_normalize_pad", dt), 0.0,
                       4.0 * net.in_ch * h * w + es * cp * in->h * in->w);
        ZJAI_HIP(launch_normalize_pad(x, net.in_ch, h, w, cp, in->h, in->w, in->v, dt, ctx.stream));
    }
    // Trunk::forward (src/model/analysis.rs:157-207)
    TensorP t = f.conv("conv1", in);
    in.reset();
    clip_after(t, 1);
    t = f.res_au("act1", t);
    ctx.check_stop();
    t = pad_for(t, 2);
    if (net.op == OP_HOP) t = f.tam("TAM", t, net.comp == COMP_Y);
    t = f.conv("conv2", t);
    clip_after(t, 2);
    t = f.res_au("act2", t);
    ctx.check_stop();
    t = pad_for(t, 4);
    if (net.op == OP_HOP) t = f.cab("cab", t);
    t = f.conv("conv3", t);
    clip_after(t, 3);
    t = f.res_au("act3", t);
    ctx.check_stop();
    if (net.comp == COMP_Y) {
        // AnalysisPrimary::forward_clip (src/model/analysis.rs:248-270)
        t = pad_for(t, 8);
        t = f.conv("conv4", t);
        clip_after(t, 4);
    }
    t = f.conv("conv5", t);
    clip_after(t, 5);
    return t;
}

void latent_decompress(Context& ctx, const Net& net, const float* res, long long res_row, long long res_plane,
                       const Windows& rwin, int H, int W, const TensorP& psi, float* y_hat) {
    if (net.kind != NET_LATENT) throw Error(ZJAI_E_INVALID_ARGUMENT, "context model: not a latent model");
    const int C = net.chs, dt = net.dtype, N = psi->n;
    if (psi->dtype != dt) throw Error(ZJAI_E_INVALID_ARGUMENT, "context model: psi precision");
    if (H <= 0 || W <= 0) throw Error(ZJAI_E_INVALID_ARGUMENT, "context model: empty residual");
    if (!net.context) {
        // upshuffle_psi_par (src/model/mcm.rs:742-746) checks
        if (psi->c != 4 * C || 2 * psi->h < H || 2 * psi->w < W)
            throw Error(ZJAI_E_INVALID_ARGUMENT, "upshuffle_psi: shape mismatch");
        LaunchScope sc(ctx, kname("k_upshuffle_psi", dt), 0.0, (double)N * C * H * W * (8.0 + dtype_size(dt)));
        ZJAI_HIP(launch_upshuffle_psi(psi->v, dt, N, C, psi->h, psi->w, res, res_row, res_plane, rwin, H, W, y_hat,
                                      ctx.stream));
        return;
    }
    const int hh = ceil_div(H, 2), hw = ceil_div(W, 2);
    if (psi->c != 4 * C || psi->h != hh || psi->w != hw)
        throw Error(ZJAI_E_INVALID_ARGUMENT, "context model: residual / psi shape mismatch");
    // STAGE_POSITIONS (src/model/mcm.rs:26): (row, column) of each stage in the 2x2 cell.
    static const int pos[4][2] = {{0, 0}, {1, 1}, {0, 1}, {1, 0}};
    Fwd f{ctx, net};
    // The reconstructed stages, concatenated along channels: stage s lands in [s C, (s + 1) C).
    TensorP stages = ctx.alloc(N, 4 * C, hh, hw, dt);
    const double es = dtype_size(dt);
    for (int s = 0; s < 4; ++s) {
        ctx.check_stop();
        const std::string p = "context.MCM." + std::to_string(s);
        TensorP psi_s = channel_view(psi, s * C, C);
        TensorP in = psi_s;
        if (s > 0) {
            TensorP t = f.conv(p + ".conv.0", channel_view(stages, 0, s * C));
            TensorP joined = ctx.alloc(N, 2 * C, hh, hw, dt);
            f.conv(p + ".conv.1", t, Epilogue{}, channel_view(joined, 0, C));
            {
                LaunchScope sc(ctx, kname("k_copy", dt), 0.0, 2.0 * es * N * C * hh * hw);
                ZJAI_HIP(launch_copy(psi_s->v, channel_view(joined, C, C)->v, dt, N, C, hh, hw, ctx.stream));
            }
            in = joined;
        }
        // FusionPredNet::forward (src/model/mcm.rs:60-66)
        Epilogue er;
        er.act = ACT_RELU;
        TensorP a = f.conv(p + ".fusion_pred_net.conv1", in, er);
        a = f.conv(p + ".fusion_pred_net.conv2", a, er);
        TensorP st = channel_view(stages, s * C, C);
        f.conv(p + ".fusion_pred_net.conv3", a, Epilogue{}, st);
        LaunchScope sc(ctx, kname("k_mcm_stage", dt), 0.0, (double)N * C * hh * hw * (2.0 * es + 8.0));
        ZJAI_HIP(launch_mcm_stage(st->v, dt, N, C, hh, hw, res, res_row, res_plane, rwin, H, W, pos[s][0], pos[s][1],
                                  y_hat, ctx.stream));
    }
}

}  // namespace zjai
