"""GPU parity of the operator layer (through the C-ABI) against the CPU oracle and the
reference's fixtures.

Tolerances (written per test):
* fp32-MFMA convolutions: max |gpu - ref| <= 1e-4 * max|ref| (the per-layer bound of the
  north-star contract); the MFMA summation order differs from the reference's serial FMA chain.
* f16 / bf16 inputs (fp32 accumulate): 4e-3 / 3e-2 * max|ref| (input rounding of 2^-11 / 2^-8).
* Elementwise ops, depthwise conv and layer norm in fp32 follow the reference's operation order
  and are required to be bit-exact.
"""

import numpy as np
import pytest

import oracle
from tests.golden import zjtb
from zenjpegai_amd import _lib, nn, synth

pytestmark = pytest.mark.gpu

TOL = {"f32": 1e-4, "f16": 4e-3, "bf16": 3e-2}


@pytest.fixture(scope="module")
def engines():
    return {p: nn.Engine(0, p) for p in ("f32", "f16", "bf16")}


@pytest.fixture(scope="module")
def igemm_engines():
    return {p: nn.Engine(0, p, flags=_lib.CTX_MFMA16_CONV3X3) for p in ("f16", "bf16")}


def rel_err(got, want):
    want = np.asarray(want, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - want)) / max(np.max(np.abs(want)), 1e-30))


def _pad_channels(x, w, groups, to=8):
    """Zero-pads input channels per group to a multiple of `to` (weights padded to match), which
    leaves the convolution's value unchanged."""
    c = x.shape[0]
    icg = c // groups
    icg_p = -(-icg // to) * to
    if icg_p == icg:
        return x, w
    xs = np.zeros((groups * icg_p,) + x.shape[1:], np.float32)
    ws = np.zeros((w.shape[0], icg_p) + w.shape[2:], np.float32)
    for g in range(groups):
        xs[g * icg_p:g * icg_p + icg] = x[g * icg:(g + 1) * icg]
    ws[:, :icg] = w
    return xs, ws


CONV_FIXTURES = [
    ("conv3x3_s1_p1_bias", 1, (1, 1), 1),
    ("conv3x3_s1_p1_g4_nobias", 1, (1, 1), 4),
    ("conv3x3_depthwise", 1, (1, 1), 12),
    ("conv1x1_nobias", 1, (0, 0), 1),
    ("conv3x3_s2_p1_bias", 2, (1, 1), 1),
    ("conv2x2_s1_p0", 1, (0, 0), 1),
]


@pytest.mark.parametrize("prec", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("name,stride,pad,groups", CONV_FIXTURES)
def test_conv_reference_fixtures(engines, prec, name, stride, pad, groups):
    eng = engines[prec]
    t = zjtb.load(name)
    x, w = t["x"], t["w"]
    if groups != x.shape[0]:
        x, w = _pad_channels(x, w, groups)
    cin = x.shape[0]
    layer = nn.ConvLayer(nn.Conv2d(cin, w.shape[0], w.shape[2:], stride, pad, groups, w,
                                   t.get("b")), eng)
    y = layer.forward(eng, nn.BTensor.from_planar(eng, x)).to_planar()
    assert y.shape == t["y"].shape
    assert rel_err(y, t["y"]) <= TOL[prec], name


@pytest.mark.parametrize("prec", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("name,pad,out_pad", [("convt4x4_s2_p1_bias", 1, 0),
                                              ("convt3x3_s2_p1_op1_bias", 1, 1)])
def test_conv_transpose_reference_fixtures(engines, prec, name, pad, out_pad):
    eng = engines[prec]
    t = zjtb.load(name)
    x, w = t["x"], t["w"]  # w [in][out][k][k]
    cin = -(-x.shape[0] // 8) * 8
    xp = np.zeros((cin,) + x.shape[1:], np.float32)
    xp[:x.shape[0]] = x
    wp = np.zeros((cin,) + w.shape[1:], np.float32)
    wp[:w.shape[0]] = w
    layer = nn.ConvTransposeLayer(nn.ConvTranspose2d(cin, w.shape[1], w.shape[2], 2, pad, out_pad,
                                                     wp, t.get("b")), eng)
    y = layer.forward(eng, nn.BTensor.from_planar(eng, xp)).to_planar()
    assert y.shape == t["y"].shape
    assert rel_err(y, t["y"]) <= TOL[prec], name


def test_unsupported_geometry_is_reported(engines):
    eng = engines["f32"]
    t = zjtb.load("conv1x3_p01_bias")
    w = np.zeros((8, 8, 1, 3), np.float32)
    with pytest.raises(_lib.HipError) as e:
        nn.ConvLayer(nn.Conv2d(8, 8, (1, 3), 1, (0, 1), 1, w), eng)
    assert e.value.kind == "Unsupported"


def _he(name, shape, fan_in, seed=11):
    return synth.normal(seed, name, shape, np.sqrt(2.0 / fan_in))


@pytest.mark.parametrize("prec", ["f32", "f16", "bf16"])
def test_config1_conv3x3_128(engines, prec):
    """BASELINE config 1 at full size (Conv2d 3x3 s1 p1 128->128 on 1x128x256x256, U[-1,1]
    input, He weights, N(0,0.01) bias); the oracle runs on the nn::fast restatement, which is
    bit-identical to the reference loops."""
    eng = engines[prec]
    x = synth.uniform(1, "cfg1/x", (128, 256, 256), -1, 1)
    w = _he("cfg1/w", (128, 128, 3, 3), 1152)
    b = synth.normal(1, "cfg1/b", (128,), 0.01)
    y = nn.ConvLayer(nn.Conv2d(128, 128, (3, 3), 1, (1, 1), 1, w, b), eng).forward(
        eng, nn.BTensor.from_planar(eng, x)).to_planar()
    want = oracle.conv2d(x, w, b, 1, (1, 1), fast=True)
    err = rel_err(y, want)
    print(f"config 1 {prec}: max |gpu - oracle| / max|oracle| = {err:.2e}")
    assert err <= TOL[prec]


DENSE16_CASES = [  # cin, cout, h, w, fused epilogue (the first four take the 8-channel store)
    (64, 64, 37, 53, "none"), (128, 128, 272, 256, "relu+add"), (128, 256, 33, 40, "leaky+gate"),
    (64, 128, 20, 24, "mul"), (128, 128, 29, 31, "sigmoid*r"), (64, 64, 20, 24, "cab")]


def _m32_width(oh, ow):
    a32 = -(-ow // 32) * 32 * (-(-oh // 8) * 8)
    a16 = -(-ow // 16) * 16 * (-(-oh // 16) * 16)
    return 16 if a16 < a32 else 32


def _takes_m32(cin, cout, h, w, n=1):
    """The runtime's choice for a dense 16-bit 3x3: conv3x3_m32 with 64 input channels, or with
    128 when its 256-position tiles number at least 256 (else conv_igemm's smaller tiles)."""
    tw = _m32_width(h, w)
    tiles = -(-w // tw) * -(-h // (256 // tw)) * n * (cout // (128 if cout % 128 == 0 else 64))
    return cin == 64 or tiles >= 256


@pytest.mark.parametrize("prec", ["f16", "bf16"])
@pytest.mark.parametrize("cin,cout,h,w,op", DENSE16_CASES)
def test_dense_16bit_conv3x3_kernels_agree(engines, igemm_engines, prec, cin, cout, h, w, op):
    """The two 16-bit dense 3x3 kernels (conv3x3_m32, 32x32x16 MFMA with the whole channel
    halo resident, and conv_igemm, 16x16x32, forced by ZJAI_CTX_MFMA16_CONV3X3) each meet the
    oracle at the precision's tolerance for every fused epilogue, on ragged sizes; the profiler
    names the kernel the runtime chose (conv3x3_m32 for 64 input channels, or for 128 when its
    tiles fill the chip)."""
    x = synth.normal(6, f"d16/x{cin}", (cin, h, w), 1.0)
    r = synth.normal(6, f"d16/r{cout}", (cout, h, w), 1.0)
    wt = _he(f"d16/w{cin}{cout}", (cout, cin, 3, 3), cin * 9)
    b = synth.normal(6, f"d16/b{cout}", (cout,), 0.05)
    base = oracle.conv2d(x, wt, b, 1, (1, 1), fast=True)
    want, kw = {
        "none": (lambda: base, {}),
        "relu+add": (lambda: oracle.add(oracle.relu(base), r), dict(act=_lib.ACT_RELU, res=_lib.RES_ADD)),
        "leaky+gate": (lambda: oracle.gate(r, oracle.leaky_relu(base)),
                       dict(act=_lib.ACT_LEAKY_RELU, res=_lib.RES_GATE)),
        "mul": (lambda: oracle.mul(r, base), dict(res=_lib.RES_MUL)),
        "sigmoid*r": (lambda: oracle.mul(r, oracle.sigmoid(base)), dict(act=_lib.ACT_SIGMOID, res=_lib.RES_MUL)),
        "cab": (lambda: oracle.add(oracle.mul(r, oracle.sigmoid(base)), x), dict(res=_lib.RES_CAB)),
    }[op]
    want = want()
    got = {}
    first = "conv3x3_m32" if _takes_m32(cin, cout, h, w) else "conv_igemm"
    for flags, kernel in ((0, first), (_lib.CTX_MFMA16_CONV3X3, "conv_igemm")):
        eng = engines[prec] if flags == 0 else igemm_engines[prec]
        layer = nn.ConvLayer(nn.Conv2d(cin, cout, (3, 3), 1, (1, 1), 1, wt, b), eng)
        xt, rt = nn.BTensor.from_planar(eng, x), nn.BTensor.from_planar(eng, r)
        if "res" in kw:
            kw = dict(kw, r1=rt, r2=xt) if op == "cab" else dict(kw, r1=rt)
        eng.sync()
        eng.profile_begin()
        y = layer.forward_fused(eng, xt, **kw)
        names = [rec[0] for rec in eng.profile_end()]
        assert any(n.startswith(kernel) for n in names), names
        got[flags] = y.to_planar()
        err = rel_err(got[flags], want)
        print(f"{prec} {cin}->{cout} {h}x{w} {op} {kernel}: {err:.2e}")
        assert err <= TOL[prec], (kernel, err)
        kw = {k: v for k, v in kw.items() if k not in ("r1", "r2")}
    assert rel_err(got[0], got[_lib.CTX_MFMA16_CONV3X3]) <= TOL[prec]


CONV1X1_CASES = [  # cin, cout, h, w, epilogue, crop (input as a cropped view)
    (128, 1024, 23, 37, "none", False), (512, 128, 19, 21, "add", False), (64, 192, 17, 40, "gate", True),
    (64, 64, 9, 14, "sigmoid*r", False), (128, 512, 13, 11, "ps2", False), (256, 64, 30, 30, "relu", True)]


@pytest.mark.parametrize("prec", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("cin,cout,h,w,op,crop", CONV1X1_CASES)
def test_conv1x1_kernels_are_bit_identical(engines, prec, cin, cout, h, w, op, crop):
    """The dedicated 1x1 GEMM kernel (conv1x1_ring: row-major position tiles, a ring of direct-LDS
    chunk loads) and the implicit-GEMM kernel (ZJAI_CTX_IGEMM_CONV1X1) give the same bits for
    every epilogue, ragged position counts and cropped input views; both meet the oracle."""
    x = synth.normal(7, f"c11/x{cin}", (cin, h + 3, w + 5) if crop else (cin, h, w), 1.0)
    r = synth.normal(7, f"c11/r{cout}", (cout, h, w), 1.0)
    wt = _he(f"c11/w{cin}{cout}", (cout, cin, 1, 1), cin)
    b = synth.normal(7, f"c11/b{cout}", (cout,), 0.05)
    xc = x[:, :h, :w]
    base = oracle.conv2d(xc, wt, b, 1, (0, 0))
    want, kw = {
        "none": (lambda: base, {}),
        "add": (lambda: oracle.add(base, r), dict(res=_lib.RES_ADD)),
        "gate": (lambda: oracle.gate(r, base), dict(res=_lib.RES_GATE)),
        "sigmoid*r": (lambda: oracle.mul(r, oracle.sigmoid(base)), dict(act=_lib.ACT_SIGMOID, res=_lib.RES_MUL)),
        "ps2": (lambda: oracle.pixel_shuffle(base, 2), dict(pixel_shuffle=2)),
        "relu": (lambda: oracle.relu(base), dict(act=_lib.ACT_RELU)),
    }[op]
    want = want()
    eng1 = nn.Engine(0, prec, flags=_lib.CTX_IGEMM_CONV1X1)
    got = []
    ring = "conv1x1_ring"
    for eng, kernel in ((engines[prec], ring), (eng1, "conv_")):
        layer = nn.ConvLayer(nn.Conv2d(cin, cout, (1, 1), 1, (0, 0), 1, wt, b), eng)
        xt = nn.BTensor.from_planar(eng, x)
        if crop:
            xt = xt.crop(h, w)
        args = dict(kw, r1=nn.BTensor.from_planar(eng, r)) if "res" in kw else kw
        eng.sync()
        eng.profile_begin()
        y = layer.forward_fused(eng, xt, **args)
        names = [rec[0] for rec in eng.profile_end()]
        assert any(n.startswith(kernel) for n in names), names
        got.append(y.to_planar())
        err = rel_err(got[-1], want)
        print(f"{prec} {cin}->{cout} {h}x{w} {op} {kernel}: {err:.2e}")
        assert err <= TOL[prec], (kernel, err)
    eng1.close()
    np.testing.assert_array_equal(got[0], got[1])


# Launch-time tile choice: (kind, cin, cout, small input h x w, large input side, expected
# kernel family on the small map). The small maps' grids are below the workgroup thresholds (narrow
# 32- / 16-channel tiles, phase-split transposed conv); the large map is the same input embedded
# top-left in zeros, whose grid takes the layer's own tile or the merged transposed kernel.
SMALL_GRID_CASES = [
    ("3x3", 192, 192, 24, 40, 256, "conv_igemm"),
    ("3x3", 192, 192, 80, 96, 256, "conv_igemm"),
    ("s2", 192, 192, 48, 80, 256, "conv_igemm"),
    ("s2", 128, 128, 48, 80, 384, "conv_igemm"),  # 16-bit large map: 128-channel tiles
    ("convT", 192, 192, 20, 24, 160, "conv_igemm"),
    ("convT", 192, 192, 80, 80, 160, "conv_igemm"),
    ("2x2", 160, 256, 64, 64, 160, "conv_igemm"),  # SOP up1 (extra pad right / bottom)
    ("2x2", 64, 128, 128, 128, 256, "conv_igemm"),  # SOP up2
]


@pytest.mark.parametrize("prec", ["f32", "bf16"])
@pytest.mark.parametrize("kind,cin,cout,h,w,big,small_kernel", SMALL_GRID_CASES)
def test_small_grid_tiles_are_bit_identical(engines, prec, kind, cin, cout, h, w, big, small_kernel):
    """A layer whose tile grid is small takes narrower tiles (or the phase-split transposed
    kernel) at launch; every tile shape sums each output in the same order, so the small map's
    output equals, bit for bit, the matching region of the same map embedded top-left in a large
    zero map (whose padding is the same zeros), which runs on the layer's default kernel."""
    eng = engines[prec]
    x = synth.uniform(11, f"sg/x{kind}{h}", (cin, h, w), -1, 1)
    xb = np.zeros((cin, big, big), np.float32)
    xb[:, :h, :w] = x
    if kind == "convT":
        wt = _he(f"sg/w{kind}", (cin, cout, 3, 3), 9 * cin)
        layer = nn.ConvTransposeLayer(nn.ConvTranspose2d(cin, cout, 3, 2, 1, 1, wt, synth.normal(11, "sg/bt", (cout,), 0.05)), eng)
        oh, ow = 2 * h, 2 * w
    elif kind == "2x2":
        wt = _he(f"sg/w{kind}", (cout, cin, 2, 2), 4 * cin)
        layer = nn.ConvLayer(nn.Conv2d(cin, cout, (2, 2), 1, (0, 0), 1, wt), eng, extra_pad=(0, 0, 1, 1))
        oh, ow = h, w
    else:
        stride = 2 if kind == "s2" else 1
        wt = _he(f"sg/w{kind}", (cout, cin, 3, 3), 9 * cin)
        layer = nn.ConvLayer(nn.Conv2d(cin, cout, (3, 3), stride, (1, 1), 1, wt, synth.normal(11, "sg/b", (cout,), 0.05)), eng)
        oh, ow = (h - 1) // stride + 1, (w - 1) // stride + 1
    outs, kernels = [], []
    for xin in (x, xb):
        xt = nn.BTensor.from_planar(eng, xin)
        eng.sync()
        eng.profile_begin()
        y = layer.forward(eng, xt)
        kernels.append([r[0] for r in eng.profile_end()][-1])
        outs.append(y.to_planar())
    print(f"{prec} {kind} {cin}->{cout} {h}x{w}: {kernels}")
    assert kernels[0].startswith(small_kernel) and kernels[0] != kernels[1], kernels
    assert outs[0].shape == (cout, oh, ow)
    np.testing.assert_array_equal(outs[0].view(np.uint32), outs[1][:, :oh, :ow].view(np.uint32))


# (cin, cout, input side, epilogue): maps whose merged grid has >= 256 workgroups, with the
# epilogues the synthesis nets put on 3x3 transposed convs (CAB upscale: RES_CAB, r1 * sigmoid(v) + r2).
CONVT_MERGED_CASES = [(160, 128, 192, "none"), (128, 128, 200, "cab"), (128, 64, 256, "add"),
                      (128, 128, 192, "leaky")]


@pytest.mark.parametrize("prec", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("cin,cout,side,epi", CONVT_MERGED_CASES)
def test_merged_transposed_conv_is_bit_identical_to_phase_split(engines, prec, cin, cout, side, epi):
    """conv_tr_merged (all four output phases per workgroup) against the phase-split kernel
    (ZJAI_CTX_PHASE_SPLIT_CONVT) on maps large enough for the merged kernel to be chosen: the same
    bits for every epilogue, and the merged output meets the oracle at the layer tolerance on the
    region a 17 x 17 input window determines."""
    x = synth.uniform(12, f"tm/x{cin}{side}", (cin, side, side - 8), -1, 1)
    wt = _he(f"tm/w{cin}{cout}", (cin, cout, 3, 3), 9 * cin)
    b = synth.normal(12, f"tm/b{cout}", (cout,), 0.05)
    oh, ow = 2 * side, 2 * (side - 8)
    r1 = synth.uniform(13, f"tm/r1{cout}{side}", (cout, oh, ow), -1, 1)
    r2 = synth.uniform(14, f"tm/r2{cout}{side}", (cout, oh, ow), -1, 1)
    split = nn.Engine(0, prec, flags=_lib.CTX_PHASE_SPLIT_CONVT)
    outs = []
    for eng, merged in ((engines[prec], True), (split, False)):
        layer = nn.ConvTransposeLayer(nn.ConvTranspose2d(cin, cout, 3, 2, 1, 1, wt, b), eng)
        kw = {"none": {}, "leaky": dict(act=_lib.ACT_LEAKY_RELU),
              "add": dict(res=_lib.RES_ADD, r1=nn.BTensor.from_planar(eng, r1)),
              "cab": dict(res=_lib.RES_CAB, r1=nn.BTensor.from_planar(eng, r1), r2=nn.BTensor.from_planar(eng, r2))}[epi]
        xt = nn.BTensor.from_planar(eng, x)
        eng.sync()
        eng.profile_begin()
        y = layer.forward_fused(eng, xt, **kw)
        names = [r[0] for r in eng.profile_end()]
        is_merged = names[-1].startswith("conv_tr_merged<")
        assert is_merged == merged and (merged or "3, 3, 1, true," in names[-1]), names
        outs.append(y.to_planar())
    split.close()
    # Oracle on the top-left 17 x 17 inputs: output rows / cols < 32 depend on no other input.
    base = oracle.conv_transpose2d(np.ascontiguousarray(x[:, :17, :17]), wt, b, 2, 1, 1)[:, :32, :32]
    q1, q2 = r1[:, :32, :32], r2[:, :32, :32]
    want = {"none": base, "leaky": oracle.leaky_relu(base),
            "add": oracle.add(base, np.ascontiguousarray(q1)),
            "cab": oracle.add(oracle.mul(np.ascontiguousarray(q1), oracle.sigmoid(base)), np.ascontiguousarray(q2))}[epi]
    err = rel_err(outs[0][:, :32, :32], want)
    print(f"{prec} convT {cin}->{cout} {side} {epi}: {err:.2e}")
    assert err <= TOL[prec]
    np.testing.assert_array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))


@pytest.mark.parametrize("prec", ["f32", "bf16"])
def test_config2_convt4_leaky(engines, prec):
    """BASELINE config 2 at full size: ConvT k4 s2 p1 192->128, 64^2 -> 128^2, then
    LeakyReLU(0.01), fused into the epilogue."""
    eng = engines[prec]
    x = synth.laplace(2, "cfg2/x", (192, 64, 64), 1.0)
    w = synth.normal(2, "cfg2/w", (192, 128, 4, 4), np.sqrt(2.0 / (192 * 4)))
    b = synth.normal(2, "cfg2/b", (128,), 0.01)
    layer = nn.ConvTransposeLayer(nn.ConvTranspose2d(192, 128, 4, 2, 1, 0, w, b), eng)
    y = layer.forward_fused(eng, nn.BTensor.from_planar(eng, x), act=_lib.ACT_LEAKY_RELU).to_planar()
    want = oracle.leaky_relu(oracle.conv_transpose2d(x, w, b, 2, 1, 0))
    assert y.shape == (128, 128, 128)
    assert rel_err(y, want) <= TOL[prec]


def config3_oracle(x, p):
    t = oracle.conv2d(x, p["c1w"], p["c1b"], 1, (1, 1), fast=True)
    t = oracle.leaky_relu(t)
    t = oracle.add(oracle.conv2d(t, p["c2w"], p["c2b"], 1, (1, 1), fast=True), x)
    g = oracle.sigmoid(oracle.conv2d(x, p["gw"], p["gb"], 1, (0, 0), fast=True))
    return oracle.mul(t, g)


def config3_params(c=192, seed=3):
    return {"c1w": _he("cfg3/c1w", (c, c, 3, 3), c * 9, seed),
            "c1b": synth.normal(seed, "cfg3/c1b", (c,), 0.01),
            "c2w": _he("cfg3/c2w", (c, c, 3, 3), c * 9, seed),
            "c2b": synth.normal(seed, "cfg3/c2b", (c,), 0.01),
            "gw": _he("cfg3/gw", (c, c, 1, 1), c, seed),
            "gb": synth.normal(seed, "cfg3/gb", (c,), 0.01)}


def config3_gpu(eng, x, p):
    c = x.shape[0]
    c1 = nn.ConvLayer(nn.Conv2d(c, c, (3, 3), 1, (1, 1), 1, p["c1w"], p["c1b"]), eng)
    c2 = nn.ConvLayer(nn.Conv2d(c, c, (3, 3), 1, (1, 1), 1, p["c2w"], p["c2b"]), eng)
    gl = nn.ConvLayer(nn.Conv2d(c, c, (1, 1), 1, (0, 0), 1, p["gw"], p["gb"]), eng)
    xt = nn.BTensor.from_planar(eng, x)
    t = c1.forward_fused(eng, xt, act=_lib.ACT_LEAKY_RELU)
    t = c2.forward_fused(eng, t, res=_lib.RES_ADD, r1=xt)
    return gl.forward_fused(eng, xt, act=_lib.ACT_SIGMOID, res=_lib.RES_MUL, r1=t)


@pytest.mark.parametrize("prec", ["f32", "bf16"])
def test_config3_residual_sigmoid_gated_block(engines, prec):
    """BASELINE config 3 at full size (t = conv3x3(leaky(conv3x3(x))) + x;
    out = t * sigmoid(conv1x1(x)), 192 channels, 1x192x128x128, U[-2,2] input)."""
    eng = engines[prec]
    x = synth.uniform(3, "cfg3/x", (192, 128, 128), -2, 2)
    p = config3_params()
    y = config3_gpu(eng, x, p).to_planar()
    err = rel_err(y, config3_oracle(x, p))
    print(f"config 3 {prec}: max |gpu - oracle| / max|oracle| = {err:.2e}")
    assert err <= TOL[prec] * 3


def test_fused_epilogues_match_op_sequences(engines):
    eng = engines["f32"]
    x = synth.normal(4, "ep/x", (64, 20, 24), 1.0)
    r = synth.normal(4, "ep/r", (64, 20, 24), 1.0)
    w = _he("ep/w", (64, 64, 3, 3), 576)
    b = synth.normal(4, "ep/b", (64,), 0.1)
    layer = nn.ConvLayer(nn.Conv2d(64, 64, (3, 3), 1, (1, 1), 1, w, b), eng)
    xt, rt = nn.BTensor.from_planar(eng, x), nn.BTensor.from_planar(eng, r)
    base = oracle.conv2d(x, w, b, 1, (1, 1))
    cases = [
        (dict(act=_lib.ACT_RELU, res=_lib.RES_ADD, r1=rt), oracle.add(oracle.relu(base), r)),
        (dict(res=_lib.RES_GATE, r1=rt), oracle.gate(r, base)),
        (dict(res=_lib.RES_CAB, r1=rt, r2=xt), oracle.add(oracle.mul(r, oracle.sigmoid(base)), x)),
        (dict(relu6_input=True), oracle.conv2d(oracle.relu6(x), w, b, 1, (1, 1))),
    ]
    for kw, want in cases:
        got = layer.forward_fused(eng, xt, **kw).to_planar()
        assert rel_err(got, want) <= 1e-4, kw
    ps = layer.forward_fused(eng, xt, pixel_shuffle=2).to_planar()
    assert rel_err(ps, oracle.pixel_shuffle(base, 2)) <= 1e-4


@pytest.mark.parametrize("cin,cout,groups", [(64, 64, 4), (32, 32, 2), (128, 128, 4), (96, 96, 6),
                                             (160, 256, 1), (144, 48, 1)])
def test_grouped_and_wide_convs(engines, cin, cout, groups):
    eng = engines["f32"]
    x = synth.normal(5, f"g/x{cin}", (cin, 19, 37), 1.0)
    w = _he(f"g/w{cin}{groups}", (cout, cin // groups, 3, 3), cin // groups * 9)
    y = nn.ConvLayer(nn.Conv2d(cin, cout, (3, 3), 1, (1, 1), groups, w), eng).forward(
        eng, nn.BTensor.from_planar(eng, x)).to_planar()
    assert rel_err(y, oracle.conv2d(x, w, None, 1, (1, 1), groups)) <= 1e-4


def test_sop_upsample_conv2x2_extra_pad(engines):
    eng = engines["f32"]
    x = synth.normal(6, "up/x", (160, 9, 13), 1.0)
    w = _he("up/w", (256, 160, 2, 2), 640)
    layer = nn.ConvLayer(nn.Conv2d(160, 256, (2, 2), 1, (0, 0), 1, w), eng, (0, 0, 1, 1))
    y = layer.forward_fused(eng, nn.BTensor.from_planar(eng, x), pixel_shuffle=2).to_planar()
    want = oracle.pixel_shuffle(oracle.conv2d(x, w, None, 1, (0, 0), 1, (0, 0, 1, 1)), 2)
    assert y.shape == want.shape == (64, 18, 26)
    assert rel_err(y, want) <= 1e-4


@pytest.mark.parametrize("k,op", [(3, 1), (4, 0)])
def test_conv_transpose_odd_sizes(engines, k, op):
    eng = engines["f32"]
    x = synth.normal(7, "t/x", (64, 7, 11), 1.0)
    w = synth.normal(7, "t/w", (64, 32, k, k), 0.1)
    b = synth.normal(7, "t/b", (32,), 0.1)
    y = nn.ConvTransposeLayer(nn.ConvTranspose2d(64, 32, k, 2, 1, op, w, b), eng).forward(
        eng, nn.BTensor.from_planar(eng, x)).to_planar()
    assert rel_err(y, oracle.conv_transpose2d(x, w, b, 2, 1, op)) <= 1e-4


@pytest.mark.parametrize("cout", [1, 2, 3, 8])
@pytest.mark.parametrize("k,op", [(3, 1), (3, 0), (4, 0)])
def test_narrow_conv_transpose_is_bit_exact(engines, cout, k, op):
    """Transposed convs with at most 8 outputs (the last synthesis layers) run on the vector ALUs
    in the reference's (input channel, tap) FMA order: in fp32 they equal the oracle bit for bit,
    here on a size that is not a multiple of the 64 x 4 workgroup tile."""
    eng = engines["f32"]
    x = synth.normal(9, "tn/x", (64, 9, 70), 1.0)
    w = synth.normal(9, "tn/w", (64, cout, k, k), 0.1)
    b = synth.normal(9, "tn/b", (cout,), 0.1)
    layer = nn.ConvTransposeLayer(nn.ConvTranspose2d(64, cout, k, 2, 1, op, w, b), eng)
    xt = nn.BTensor.from_planar(eng, x)
    y = layer.forward(eng, xt).to_planar()
    want = oracle.conv_transpose2d(x, w, b, 2, 1, op)
    assert y.shape == want.shape
    assert np.array_equal(y, want)
    # relu6 on load (ResAU's input clamp) goes through the same kernel.
    y6 = layer.forward_fused(eng, xt, relu6_input=True).to_planar()
    assert np.array_equal(y6, oracle.conv_transpose2d(oracle.relu6(x), w, b, 2, 1, op))


def _round_storage(a, prec):
    """IEEE round-to-nearest-even of f32 values to the 16-bit storage type, back in f32."""
    a = np.ascontiguousarray(a, np.float32)
    if prec == "f16":
        return a.astype(np.float16).astype(np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


@pytest.mark.parametrize("prec", ["f16", "bf16"])
@pytest.mark.parametrize("cout,op", [(1, 1), (2, 0)])
def test_narrow_conv_transpose_3x3_16bit_is_exact(engines, prec, cout, op):
    """The 3x3 narrow transposed conv on the vector ALUs (k_convT3_narrow, selected by
    ZJAI_CTX_VALU_NARROW_CONVT in the 16-bit precisions) computes in f32 on the stored (rounded)
    inputs and weights in the reference's FMA order, so its output is the oracle's f32 result on
    those rounded operands, rounded once to the storage type -- bit for bit. 128 input channels
    (two 128-byte chunks in 16-bit), a map not a multiple of the tile."""
    eng = nn.Engine(0, prec, flags=_lib.CTX_VALU_NARROW_CONVT)
    x = synth.normal(11, "t3/x", (128, 19, 45), 1.0)
    w = synth.normal(11, f"t3/w{cout}", (128, cout, 3, 3), 0.1)
    b = synth.normal(11, f"t3/b{cout}", (cout,), 0.1)
    layer = nn.ConvTransposeLayer(nn.ConvTranspose2d(128, cout, 3, 2, 1, op, w, b), eng)
    eng.sync()
    eng.profile_begin()
    y = layer.forward(eng, nn.BTensor.from_planar(eng, x)).to_planar()
    names = [r[0] for r in eng.profile_end()]
    eng.close()
    assert any(n.startswith("k_convT3_narrow") for n in names), names
    want = _round_storage(oracle.conv_transpose2d(_round_storage(x, prec), _round_storage(w, prec), b, 2, 1, op),
                          prec)
    assert np.array_equal(y, want)


# (cin, cout, output padding, input h x w): HOP luma's last layer (128 -> 1), HOP chroma's
# (64 -> 8), and 2 / 4 outputs (one 16-row block of (phase, output) rows, partly or fully used).
MFMA_NARROW_CASES = [(128, 1, 1, 19, 45), (64, 8, 1, 23, 37), (128, 2, 0, 17, 33), (64, 4, 1, 9, 70)]


@pytest.mark.parametrize("prec", ["f16", "bf16"])
@pytest.mark.parametrize("cin,cout,op,h,w", MFMA_NARROW_CASES)
def test_narrow_conv_transpose_3x3_16bit_mfma(engines, prec, cin, cout, op, h, w):
    """The default 16-bit form of the same layers (k_convT3_mfma: one GEMM per phase-grid position
    over the 2 x 2 input neighbourhood, 16x16x32 MFMAs) sums the same exact f32 products as the
    vector kernel in another order: against the oracle's f32 result on the rounded operands,
    rounded to the storage type, it is within two storage ulps of the largest output everywhere
    (f16 2 x 2^-11, bf16 2 x 2^-8 of max|oracle|) and equal in most samples; relu6 on load too."""
    eng = engines[prec]
    x = synth.normal(16, f"tm16/x{cin}", (cin, h, w), 1.0)
    wt = synth.normal(16, f"tm16/w{cin}{cout}", (cin, cout, 3, 3), 0.1)
    b = synth.normal(16, f"tm16/b{cout}", (cout,), 0.1)
    layer = nn.ConvTransposeLayer(nn.ConvTranspose2d(cin, cout, 3, 2, 1, op, wt, b), eng)
    xr, wr = _round_storage(x, prec), _round_storage(wt, prec)
    bound = 2.0 * (2.0 ** -11 if prec == "f16" else 2.0 ** -8)
    for relu6 in (False, True):
        eng.sync()
        eng.profile_begin()
        y = layer.forward_fused(eng, nn.BTensor.from_planar(eng, x), relu6_input=relu6).to_planar()
        names = [r[0] for r in eng.profile_end()]
        assert any(n.startswith("k_convT3_mfma") for n in names), names
        want = _round_storage(oracle.conv_transpose2d(oracle.relu6(xr) if relu6 else xr, wr, b, 2, 1, op), prec)
        assert y.shape == want.shape
        err = rel_err(y, want)
        same = float(np.mean(y == want))
        print(f"{prec} {cin}->{cout} op {op} relu6 {relu6}: rel err {err:.2e}, equal {same:.4f}")
        assert err <= bound and same >= 0.9, (err, same)


@pytest.mark.parametrize("prec", ["f16", "bf16"])
def test_narrow_conv_transpose_fast_paths(engines, prec):
    eng = engines[prec]
    x = synth.normal(10, "tn/x", (64, 12, 20), 1.0)
    w = synth.normal(10, "tn/w", (64, 8, 3, 3), 0.1)
    b = synth.normal(10, "tn/b", (8,), 0.1)
    y = nn.ConvTransposeLayer(nn.ConvTranspose2d(64, 8, 3, 2, 1, 1, w, b), eng).forward(
        eng, nn.BTensor.from_planar(eng, x)).to_planar()
    assert rel_err(y, oracle.conv_transpose2d(x, w, b, 2, 1, 1)) <= TOL[prec]


def test_elementwise_ops_are_bit_exact(engines):
    eng = engines["f32"]
    a = synth.normal(8, "el/a", (16, 9, 10), 3.0)
    b = synth.normal(8, "el/b", (16, 9, 10), 1.0)
    for fn, ref in [(nn.relu, oracle.relu), (nn.relu6, oracle.relu6), (nn.leaky_relu, oracle.leaky_relu),
                    (nn.sigmoid, oracle.sigmoid)]:
        t = nn.BTensor.from_planar(eng, a)
        fn(eng, t)
        assert np.array_equal(t.to_planar().view(np.uint32), ref(a).view(np.uint32)), fn.__name__
    for fn, ref in [(nn.add_assign, oracle.add), (nn.gate, oracle.gate), (nn.mul_assign, oracle.mul),
                    (nn.elu_gate, oracle.elu_gate)]:
        t = nn.BTensor.from_planar(eng, a)
        fn(eng, t, nn.BTensor.from_planar(eng, b))
        assert np.array_equal(t.to_planar().view(np.uint32), ref(a, b).view(np.uint32)), fn.__name__
    ps = nn.pixel_shuffle(eng, nn.BTensor.from_planar(eng, synth.normal(8, "el/p", (64, 3, 5))), 2)
    assert np.array_equal(ps.to_planar(), oracle.pixel_shuffle(synth.normal(8, "el/p", (64, 3, 5)), 2))


def test_depthwise_and_layer_norm_are_bit_exact(engines):
    eng = engines["f32"]
    x = synth.normal(9, "dw/x", (384, 11, 13), 1.0)
    w = synth.normal(9, "dw/w", (384, 1, 3, 3), 0.3)
    y = nn.ConvLayer(nn.Conv2d(384, 384, (3, 3), 1, (1, 1), 384, w), eng).forward(
        eng, nn.BTensor.from_planar(eng, x)).to_planar()
    assert np.array_equal(y.view(np.uint32), oracle.conv2d(x, w, None, 1, (1, 1), 384).view(np.uint32))
    lw = synth.normal(9, "ln/w", (128,), 1.0)
    lb = synth.normal(9, "ln/b", (128,), 1.0)
    xl = synth.normal(9, "ln/x", (128, 7, 9), 2.0)
    got = nn.layer_norm_channels(eng, nn.BTensor.from_planar(eng, xl), lw, lb).to_planar()
    assert np.array_equal(got.view(np.uint32), oracle.layer_norm_channels(xl, lw, lb).view(np.uint32))


# (dim, heads, h, w, cropped view). Besides the synthesis nets' shapes (4 heads, dim 128 / 64)
# these reach the Gram kernel's other paths: more than four heads (two head groups), a sub-chunk
# needing more than one round of loads (dim 256), 12 channels per head (one 16-channel block),
# and a cropped view (rows wider than the map: per-unit addresses).
ATTENTION_CASES = [(128, 4, 24, 40, False), (64, 4, 33, 17, False), (128, 8, 21, 30, False),
                   (256, 8, 20, 26, False), (48, 4, 19, 23, False), (128, 4, 24, 40, True)]


@pytest.mark.parametrize("prec", ["f32", "bf16"])
@pytest.mark.parametrize("dim,heads,h,w,crop", ATTENTION_CASES)
def test_channel_attention(engines, prec, dim, heads, h, w, crop):
    """Channel attention through the C-ABI against the oracle: 1e-5 of the largest output in
    f32 (the reference normalises q and k before its dot, the kernels divide the raw dot by the
    norms after); in bf16 against the oracle on the rounded input, 1e-2 (the output's own
    rounding is 2^-9)."""
    eng = engines[prec]
    hh, ww = (h + 3, w + 5) if crop else (h, w)
    qkv = synth.normal(10, f"at/{dim}/{heads}", (3 * dim, hh, ww), 1.0)
    temp = np.linspace(0.7, 2.0, heads).astype(np.float32)
    t = nn.BTensor.from_planar(eng, qkv)
    if crop:
        t = t.crop(h, w)
    got = nn.channel_attention(eng, t, heads, temp).to_planar()
    q = np.ascontiguousarray(qkv[:, :h, :w])
    if prec != "f32":
        q = _round_storage(q, prec)
    err = rel_err(got, oracle.channel_attention(q, heads, temp))
    print(f"{prec} dim {dim} heads {heads} {h}x{w} crop {crop}: {err:.2e}")
    assert err <= (1e-5 if prec == "f32" else 1e-2)


def test_attention_one_position_kat(engines):
    """src/nn/fast/math.rs:936-943 through the HIP path (dim padded to 8 with zero rows)."""
    eng = engines["f32"]
    q = np.zeros((24, 1, 1), np.float32)
    # head 0 of 4: q rows (2, -3)... embed the KAT in channels 0-1 of each of q, k, v.
    # With 4 heads of 2 channels: head 0 holds the KAT, the other heads are zeros.
    q[0:2, 0, 0] = [2.0, -3.0]
    q[8:10, 0, 0] = [0.5, 4.0]
    q[16:18, 0, 0] = [10.0, 20.0]
    got = nn.channel_attention(eng, nn.BTensor.from_planar(eng, q), 4, np.ones(4, np.float32)).to_planar()
    assert got[0:2, 0, 0].tolist() == [15.0, 15.0]


@pytest.mark.parametrize("prec", ["f32", "bf16"])
def test_new_tensors_are_zero_at_any_byte_size(engines, prec):
    """zjai_tensor_create clears its buffer with the zero-fill kernel (no hipMemsetAsync, so a
    capturing caller may create tensors), on odd map sizes too. The first tensor's nonzero buffer
    goes back to the pool and is handed out again to the second."""
    eng = engines[prec]
    for c, h, w in ((4, 5, 7), (8, 3, 3), (4, 1, 1)):
        t = nn.BTensor.from_planar(eng, np.full((c, h, w), 3.0, np.float32))
        del t
        eng.sync()
        z = nn.BTensor.zeros(eng, c, h, w)
        assert not np.any(z.to_planar()), (c, h, w)


def test_tensors_and_layers_may_outlive_their_context():
    """Destroying the context first is allowed: tensors return their blocks to the pool they
    share with it (which lives until the last of them), layers free their own weights."""
    eng = nn.Engine(0, "f32")
    x = nn.BTensor.from_planar(eng, synth.normal(13, "life/x", (16, 6, 7), 1.0))
    layer = nn.ConvLayer(nn.Conv2d(16, 16, (3, 3), 1, (1, 1), 1,
                                   synth.normal(13, "life/w", (16, 16, 3, 3), 0.1)), eng)
    y = layer.forward(eng, x)
    eng.sync()
    eng.close()
    del x, y, layer
    eng2 = nn.Engine(0, "f32")
    z = nn.BTensor.from_planar(eng2, np.ones((8, 3, 3), np.float32))
    assert np.array_equal(z.to_planar(), np.ones((8, 3, 3), np.float32))
