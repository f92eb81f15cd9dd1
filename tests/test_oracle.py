"""Pins the CPU oracle (test infrastructure) against the reference's own golden vectors and KATs,
and against what the mathematics fixes (independent formulations, closed forms, brute force).
CPU only."""

import math
from fractions import Fraction

import numpy as np
import pytest

import oracle
from oracle import geometry as geo
from tests.golden import zjtb

rng = np.random.default_rng(1234)


def _close_rel(got, want, tol):
    """The reference's fixture metric: max |g - w| / max(|w|, 1) (tests/nn_vectors.rs:55-62)."""
    assert got.shape == want.shape
    err = np.max(np.abs(got.astype(np.float64) - want) / np.maximum(np.abs(want), 1.0))
    assert err < tol, err


# ------------------------------------------------------------------------ reference fixtures
CONV_CASES = [
    ("conv3x3_s1_p1_bias", 1, (1, 1), 1),
    ("conv3x3_s1_p1_g4_nobias", 1, (1, 1), 4),
    ("conv3x3_depthwise", 1, (1, 1), 12),
    ("conv1x1_nobias", 1, (0, 0), 1),
    ("conv3x3_s2_p1_bias", 2, (1, 1), 1),
    ("conv2x2_s1_p0", 1, (0, 0), 1),
    ("conv1x3_p01_bias", 1, (0, 1), 1),
    ("conv3x1_p10_bias", 1, (1, 0), 1),
]


@pytest.mark.parametrize("name,stride,pad,groups", CONV_CASES)
def test_conv2d_matches_reference_fixture(name, stride, pad, groups):
    t = zjtb.load(name)
    y = oracle.conv2d(t["x"], t["w"], t.get("b"), stride, pad, groups)
    _close_rel(y, t["y"], 2e-6)


@pytest.mark.parametrize("name,pad,out_pad", [("convt4x4_s2_p1_bias", 1, 0),
                                              ("convt3x3_s2_p1_op1_bias", 1, 1)])
def test_conv_transpose2d_matches_reference_fixture(name, pad, out_pad):
    t = zjtb.load(name)
    y = oracle.conv_transpose2d(t["x"], t["w"], t.get("b"), 2, pad, out_pad)
    _close_rel(y, t["y"], 2e-6)


def test_pixel_shuffle_matches_reference_fixture_exactly():
    t = zjtb.load("pixel_shuffle")
    for r, key in ((2, "y2"), (4, "y4")):
        y = oracle.pixel_shuffle(t["x"], r)
        assert y.shape == t[key].shape
        assert np.array_equal(y.view(np.uint32), t[key].view(np.uint32))


# ------------------------------------------------------------------ independent formulations
def _np_conv(x, w, b, stride, pad, groups, extra=(0, 0, 0, 0)):
    """Gather formulation in float64 (a different algorithm from the oracle's loops)."""
    x = np.pad(x.astype(np.float64), ((0, 0), (extra[0] + pad[0], extra[2] + pad[0]),
                                      (extra[1] + pad[1], extra[3] + pad[1])))
    oc, icg, kh, kw = w.shape
    oh = (x.shape[1] - kh) // stride + 1
    ow = (x.shape[2] - kw) // stride + 1
    out = np.zeros((oc, oh, ow))
    ocg = oc // groups
    for g in range(groups):
        xs = x[g * icg:(g + 1) * icg]
        for ky in range(kh):
            for kx in range(kw):
                patch = xs[:, ky:ky + stride * oh:stride, kx:kx + stride * ow:stride]
                out[g * ocg:(g + 1) * ocg] += np.einsum(
                    "oi,ihw->ohw", w[g * ocg:(g + 1) * ocg, :, ky, kx].astype(np.float64), patch)
    if b is not None:
        out += b[:, None, None]
    return out


def _np_convt(x, w, b, stride, pad, out_pad):
    """Scatter formulation: in[ic, y, x] contributes to out[s*y - pad + ky, s*x - pad + kx]."""
    ic, oc, k, _ = w.shape
    h, wd = x.shape[1:]
    oh = (h - 1) * stride + k + out_pad - 2 * pad
    ow = (wd - 1) * stride + k + out_pad - 2 * pad
    big = np.zeros((oc, (h - 1) * stride + k + stride, (wd - 1) * stride + k + stride))
    for ky in range(k):
        for kx in range(k):
            contrib = np.einsum("io,ihw->ohw", w[:, :, ky, kx].astype(np.float64),
                                x.astype(np.float64))
            big[:, ky:ky + stride * h:stride, kx:kx + stride * wd:stride] += contrib
    out = big[:, pad:pad + oh, pad:pad + ow]
    if b is not None:
        out = out + b[:, None, None]
    return out


@pytest.mark.parametrize("c,oc,k,stride,pad,groups,extra", [
    (8, 6, 3, 1, 1, 1, (0, 0, 0, 0)),
    (16, 16, 3, 1, 1, 4, (0, 0, 0, 0)),
    (12, 12, 3, 1, 1, 12, (0, 0, 0, 0)),
    (10, 7, 1, 1, 0, 1, (0, 0, 0, 0)),
    (5, 8, 3, 2, 1, 1, (0, 0, 0, 0)),
    (6, 8, 2, 1, 0, 1, (0, 0, 1, 1)),
    (32, 20, 3, 2, 1, 2, (1, 0, 2, 1)),
])
def test_conv2d_equals_gather_formulation(c, oc, k, stride, pad, groups, extra):
    x = rng.standard_normal((c, 9, 11)).astype(np.float32)
    w = rng.standard_normal((oc, c // groups, k, k)).astype(np.float32)
    b = rng.standard_normal(oc).astype(np.float32)
    y = oracle.conv2d(x, w, b, stride, (pad, pad), groups, extra)
    want = _np_conv(x, w, b, stride, (pad, pad), groups, extra)
    assert y.shape == want.shape
    assert np.max(np.abs(y - want)) < 1e-4 * max(1.0, np.max(np.abs(want)))


@pytest.mark.parametrize("k,pad,out_pad", [(4, 1, 0), (3, 1, 1), (3, 0, 0), (4, 2, 1)])
def test_conv_transpose2d_equals_scatter_formulation(k, pad, out_pad):
    x = rng.standard_normal((5, 6, 7)).astype(np.float32)
    w = rng.standard_normal((5, 4, k, k)).astype(np.float32)
    b = rng.standard_normal(4).astype(np.float32)
    y = oracle.conv_transpose2d(x, w, b, 2, pad, out_pad)
    want = _np_convt(x, w, b, 2, pad, out_pad)
    assert y.shape == want.shape
    assert np.max(np.abs(y - want)) < 1e-4 * max(1.0, np.max(np.abs(want)))


def test_conv1x1_is_a_matmul():
    x = rng.standard_normal((24, 5, 6)).astype(np.float32)
    w = rng.standard_normal((10, 24, 1, 1)).astype(np.float32)
    y = oracle.conv2d(x, w, None)
    want = (w[:, :, 0, 0].astype(np.float64) @ x.reshape(24, -1).astype(np.float64)).reshape(10, 5, 6)
    assert np.max(np.abs(y - want)) < 1e-4


def _round_f32(fr: Fraction) -> np.float32:
    """Correctly rounded (RNE) float32 of an exact rational."""
    c = np.float32(float(fr))
    cands = [np.nextafter(c, np.float32(-np.inf)), c, np.nextafter(c, np.float32(np.inf))]
    best = min(cands, key=lambda v: (abs(Fraction(float(v)) - fr),
                                     int(np.float32(v).view(np.uint32)) & 1))
    return np.float32(best)


def _fma(a, b, c):
    return _round_f32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def test_conv2d_follows_the_contract_order_bit_for_bit():
    """acc = bias; for ic { for ky { for kx { acc = fma(w, x, acc) } } }, padding taps included
    (src/nn/mod.rs:12-13), checked with exact rational arithmetic on a tiny case."""
    x = (rng.standard_normal((3, 4, 4)) * 3).astype(np.float32)
    w = rng.standard_normal((2, 3, 3, 3)).astype(np.float32)
    b = rng.standard_normal(2).astype(np.float32)
    y = oracle.conv2d(x, w, b, 1, (1, 1))
    xp = np.pad(x, ((0, 0), (1, 1), (1, 1)))
    for oc in range(2):
        for oy in range(4):
            for ox in range(4):
                acc = b[oc]
                for ic in range(3):
                    for ky in range(3):
                        for kx in range(3):
                            acc = _fma(w[oc, ic, ky, kx], xp[ic, oy + ky, ox + kx], acc)
                assert y[oc, oy, ox].view(np.uint32) == np.float32(acc).view(np.uint32)


def test_conv_transpose_follows_the_contract_order_bit_for_bit():
    x = (rng.standard_normal((2, 3, 3)) * 3).astype(np.float32)
    w = rng.standard_normal((2, 2, 3, 3)).astype(np.float32)
    b = rng.standard_normal(2).astype(np.float32)
    y = oracle.conv_transpose2d(x, w, b, 2, 1, 1)
    for oc in range(2):
        for oy in range(6):
            for ox in range(6):
                acc = b[oc]
                for ic in range(2):
                    for ky in range(3):
                        if (oy + 1 - ky) % 2:
                            continue
                        iy = (oy + 1 - ky) // 2
                        for kx in range(3):
                            if (ox + 1 - kx) % 2:
                                continue
                            ix = (ox + 1 - kx) // 2
                            xv = x[ic, iy, ix] if 0 <= iy < 3 and 0 <= ix < 3 else np.float32(0)
                            acc = _fma(w[ic, oc, ky, kx], xv, acc)
                assert y[oc, oy, ox].view(np.uint32) == np.float32(acc).view(np.uint32)


def test_pixel_shuffle_roundtrip_index_map():
    x = np.arange(8 * 3 * 5, dtype=np.float32).reshape(8, 3, 5)
    y = oracle.pixel_shuffle(x, 2)
    # torch's definition: view (c, r, r, h, w) -> permute (c, h, r, w, r)
    want = x.reshape(2, 2, 2, 3, 5).transpose(0, 3, 1, 4, 2).reshape(2, 6, 10)
    assert np.array_equal(y, want)


# ------------------------------------------------------------------------ elementwise math
def test_exp_tracks_libm_and_kat():
    """KAT of src/nn/fast/math.rs:921-934."""
    xs = np.arange(-87.0, 88.0, 0.0037, dtype=np.float64).astype(np.float32)
    got = oracle.exp(xs).astype(np.float64)
    want = np.exp(xs.astype(np.float64))
    assert np.max(np.abs((got - want) / want)) < 3e-7
    L = oracle.lib()
    assert L.or_exp(0.0) == 1.0
    assert 0.0 < L.or_exp(-1000.0) < 2e-38
    assert math.isnan(L.or_exp(float("nan")))


def test_sigmoid_and_elu_gate():
    x = np.linspace(-30, 30, 2001, dtype=np.float32)
    s = oracle.sigmoid(x).astype(np.float64)
    assert np.max(np.abs(s - 1 / (1 + np.exp(-x.astype(np.float64))))) < 1e-6
    assert oracle.sigmoid(np.zeros(1, np.float32))[0] == 0.5
    g = rng.standard_normal(x.size).astype(np.float32)
    e = oracle.elu_gate(x, g).astype(np.float64)
    xd = x.astype(np.float64)
    want = np.where(xd > 0, xd, np.expm1(xd)) * g
    assert np.max(np.abs(e - want)) < 1e-5


def test_gate_is_two_ieee_ops_not_an_fma():
    x = np.float32(1.0000001) * np.ones(4, np.float32)
    m = np.array([1e-7, 3e-8, -0.5, 2.0], np.float32)
    got = oracle.gate(x, m)
    want = (x * (np.float32(1) + m)).astype(np.float32)  # numpy: separate roundings
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_relu_relu6_leaky_denormalize_closed_forms():
    x = np.array([-3.0, -0.0, 0.5, 7.0, 300.0, -1e-3], np.float32)
    assert np.array_equal(oracle.relu(x), np.maximum(x, 0))
    assert np.array_equal(oracle.relu6(x), np.clip(x, 0, 6))
    assert np.array_equal(oracle.leaky_relu(x), np.where(x < 0, x * np.float32(0.01), x))
    d = oracle.denormalize(x)
    assert np.array_equal(d, np.clip(x * np.float32(128) + np.float32(127.5), 0, 255))


def test_quantize_plane_round_half_even():
    # 8-bit: x/255*255 is x (exact for integers) -> rint of half-integers goes to even.
    x = np.array([-1, 0, 0.5, 1.5, 2.5, 254.5, 255, 300, 127.49], np.float32)
    q = oracle.quantize_plane(x, 8)
    assert q.tolist() == [0, 0, 0, 2, 2, 254, 255, 255, 127]
    # 10-bit: closed form with float32 ops.
    v = rng.uniform(-5, 260, 4096).astype(np.float32)
    q10 = oracle.quantize_plane(v, 10)
    c = np.clip(v, 0, 255)
    want = np.clip(np.rint((c / np.float32(255)) * np.float32(1023)), 0, 1023).astype(np.uint16)
    assert np.array_equal(q10, want)


# ---------------------------------------------------------------------- layer norm / attention
def test_layer_norm_matches_f64_definition():
    x = rng.standard_normal((24, 5, 7)).astype(np.float32) * 3 + 1
    wt = rng.standard_normal(24).astype(np.float32)
    bs = rng.standard_normal(24).astype(np.float32)
    y = oracle.layer_norm_channels(x, wt, bs)
    xd = x.astype(np.float64)
    mean = xd.mean(0)
    var = ((xd - mean) ** 2).mean(0)
    want = (xd - mean) / np.sqrt(var + 1e-5) * wt[:, None, None] + bs[:, None, None]
    assert np.max(np.abs(y - want)) < 1e-5


def test_attention_of_one_position_is_value_mix():
    """KAT of src/nn/fast/math.rs:936-943."""
    qkv = np.array([2.0, -3.0, 0.5, 4.0, 10.0, 20.0], np.float32).reshape(6, 1, 1)
    out = oracle.channel_attention(qkv, 1, np.array([1.0], np.float32))
    assert out.ravel().tolist() == [15.0, 15.0]


def test_channel_attention_matches_brute_force():
    dim, heads, h, w = 16, 4, 6, 7
    qkv = rng.standard_normal((3 * dim, h, w)).astype(np.float32)
    temp = np.array([0.5, 1.0, 2.0, 3.0], np.float32)
    out, attn = oracle.channel_attention(qkv, heads, temp, return_attn=True)
    c = dim // heads
    q = qkv[:dim].reshape(dim, -1).astype(np.float64)
    k = qkv[dim:2 * dim].reshape(dim, -1).astype(np.float64)
    v = qkv[2 * dim:].reshape(dim, -1).astype(np.float64)
    q /= np.maximum(np.linalg.norm(q, axis=1, keepdims=True), 1e-12)
    k /= np.maximum(np.linalg.norm(k, axis=1, keepdims=True), 1e-12)
    want = np.zeros((dim, h * w))
    for hd in range(heads):
        s = slice(hd * c, (hd + 1) * c)
        a = q[s] @ k[s].T * temp[hd]
        a = np.exp(a - a.max(1, keepdims=True))
        a /= a.sum(1, keepdims=True)
        assert np.max(np.abs(attn[s] - a)) < 1e-6
        want[s] = a @ v[s]
    assert np.max(np.abs(out.reshape(dim, -1) - want)) < 1e-5


def test_dot8_pairwise_order():
    a = np.array([1e16, 1, -1e16, 1, 0, 0, 0, 0, 3], np.float32)
    b = np.ones(9, np.float32)
    # lanes: acc0 = 1e16 + 3, acc1 = 1, acc2 = -1e16, acc3 = 1 -> ((acc0+acc1)+(acc2+acc3))
    acc = [np.float64(0)] * 8
    for i in range(9):
        acc[i % 8] += np.float64(a[i])
    want = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]))
    assert oracle.dot8(a, b) == want


# ------------------------------------------------------------------------------ f16 rounding
def test_f16_upcast_is_exact_for_every_half():
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_bits_to_f32(int(h)) for h in bits], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f16_rounding_is_ieee_rne():
    """The reference's integer algorithm (src/weights/f16.rs:12-53) equals IEEE RNE, which
    numpy's float16 cast implements: checked on random and edge values."""
    v = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 20000),
        np.array([65504, 65519.99, 65520, 1e-8, 2.98e-8, 2.9802322e-8, 5.96e-8, -0.0, np.inf,
                  -np.inf, 6.1035156e-05, 6.1e-05], np.float32)]).astype(np.float32)
    got = np.array([oracle.f32_to_f16_bits(float(x)) for x in v], np.uint16)
    want = v.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    rt = oracle.f16_round_trip(v)
    assert np.array_equal(rt, v.astype(np.float16).astype(np.float32))


# --------------------------------------------------------------------------------- geometry
def test_tiles_disabled_is_one_tile():
    t = geo.synthesis_tiles(888, 560, 56, 35)
    assert len(t) == 1 and t[0].core == geo.Area(0, 0, 560, 888)


def test_tiles_match_reference_layout():
    """KAT of src/tools/tiles.rs:489-520 (reference log, 2096x1400, tile 1024, overlap 64)."""
    t = geo.synthesis_tiles(1400, 2096, 88, 131, (1024, 64))
    A = geo.Area
    assert [x.image for x in t] == [A(0, 0, 1024, 1024), A(960, 0, 1024, 1024),
                                   A(1920, 0, 176, 1024), A(0, 960, 1024, 440),
                                   A(960, 960, 1024, 440), A(1920, 960, 176, 440)]
    assert t[1].latent == A(60, 0, 64, 64)
    assert t[5].latent == A(120, 60, 11, 28)
    assert t[1].core == A(992, 0, 960, 992) and t[1].core_offset == (32, 0)
    assert t[5].core == A(1952, 992, 144, 408)
    assert sum(x.core.width * x.core.height for x in t) == 1400 * 2096


def test_tiles_match_reference_layout_with_independent_regions():
    """KAT of src/tools/tiles.rs:522-556."""
    A = geo.Area
    regions = geo.RegionGrid(1, 2, (A(0, 0, 1024, 1400), A(1024, 0, 1072, 1400)),
                             (A(0, 0, 1024, 1400), A(1024, 0, 1072, 1400)))
    t = geo.synthesis_tiles(1400, 2096, 88, 131, (640, 128), regions)
    assert [x.image for x in t] == [
        A(0, 0, 704, 704), A(640, 0, 640, 640), A(1216, 0, 768, 704), A(1856, 0, 240, 704),
        A(0, 576, 704, 768), A(640, 640, 640, 640), A(1216, 576, 768, 768),
        A(1856, 576, 240, 768), A(0, 1216, 704, 184), A(640, 1280, 640, 120),
        A(1216, 1216, 768, 184), A(1856, 1216, 240, 184)]
    assert t[6].latent == A(76, 36, 48, 48)
    assert t[6].core == A(1280, 640, 640, 640) and t[6].core_offset == (64, 64)
    assert sum(x.core.width * x.core.height for x in t) == 1400 * 2096


def test_tiles_reject_degenerate_headers():
    with pytest.raises(geo.GeometryError):
        geo.synthesis_tiles(1400, 2096, 88, 131, (64, 64))


def test_region_axis_and_grid_kats():
    """KATs of src/tools/regions.rs:151-181."""
    assert geo.axis_coords(888, 1, 4, False) == [(0, 56)]
    assert geo.axis_coords(560, 1, 6, False) == [(0, 9)]
    assert geo.axis_coords(3000, 3, 4, True) == [(0, 64), (64, 128), (128, 188)]
    assert geo.axis_coords(3000, 3, 6, True) == [(0, 16), (16, 32), (32, 47)]
    g = geo.grid([(0, 64), (64, 128), (128, 188)], [(0, 100), (100, 250)], 4)
    A = geo.Area
    assert g[0] == A(0, 0, 104, 68) and g[1] == A(96, 0, 154, 68)
    assert g[2] == A(0, 60, 104, 72) and g[5] == A(96, 124, 154, 64)


def test_4k_independent_region_tiling_is_24_tiles():
    """Config 5 geometry: 3840x2160, 2x3 independent regions, tile 640 / overlap 128."""
    assert geo.region_counts(2160, 3840) == (2, 3)
    assert geo.synthesis_tiling(2160, 3840, (2, 3)) == (640, 128)
    regions = geo.image_region_grid(2160, 3840, 2, 3)
    assert [a.x for a in regions.core[:3]] == [0, 1280, 2560]
    assert [a.y for a in regions.core[::3]] == [0, 1024]
    t = geo.synthesis_tiles(2160, 3840, 135, 240, (640, 128), regions)
    assert len(t) == 24
    assert sum(x.core.width * x.core.height for x in t) == 2160 * 3840
    shapes = sorted({(x.image.width, x.image.height) for x in t})
    assert (640, 640) in shapes or (704, 704) in shapes


# ------------------------------------------------- nn::fast restatement (the CPU baseline)
def _tiers():
    tiers = [8]
    try:
        oracle.force_cpu_tier(16)
        tiers.append(16)
    except oracle.OracleError:
        pass
    finally:
        oracle.force_cpu_tier(0)
    return tiers


@pytest.fixture(params=_tiers())
def cpu_tier(request):
    oracle.force_cpu_tier(request.param)
    yield request.param
    oracle.force_cpu_tier(0)


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


@pytest.mark.parametrize("c,oc,k,stride,pad,groups,extra,h,w", [
    (128, 128, 3, 1, 1, 1, (0, 0, 0, 0), 13, 50),    # HOP residual conv, a tail block per row
    (20, 36, 3, 1, 1, 1, (0, 0, 0, 0), 7, 29),       # partial input / output blocks
    (128, 128, 3, 2, 1, 1, (0, 0, 0, 0), 17, 33),    # CAB / TAM stride-2 conv
    (128, 128, 3, 1, 1, 4, (0, 0, 0, 0), 10, 27),    # ResAU grouped conv (32 per group)
    (64, 64, 1, 1, 0, 1, (0, 0, 0, 0), 5, 60),       # 1x1
    (144, 128, 2, 1, 0, 1, (0, 0, 1, 1), 6, 9),      # SOP upsampler 2x2 with extra pad
    (64, 64, 3, 1, 1, 4, (0, 0, 0, 0), 6, 7),        # 16 per group: the oracle-loop fallback
    (256, 48, 3, 1, 1, 1, (0, 0, 0, 0), 8, 8),       # combine layer
    (384, 384, 3, 1, 1, 384, (0, 0, 0, 0), 11, 37),  # depthwise (prep_data conv2)
    (24, 24, 3, 1, 1, 24, (1, 0, 0, 2), 5, 9),       # depthwise with extra pad
    (16, 16, 2, 1, 0, 16, (0, 0, 1, 1), 4, 3),       # depthwise 2x2
])
def test_fast_conv2d_equals_reference_loops_bit_for_bit(cpu_tier, c, oc, k, stride, pad, groups,
                                                        extra, h, w):
    """nn::fast is bit-identical to nn::reference by contract (src/nn/mod.rs:1-29,
    tests/fast_vs_reference.rs); so is its restatement, in both SIMD tiers."""
    x = rng.standard_normal((c, h, w)).astype(np.float32)
    wt = (rng.standard_normal((oc, c // groups, k, k)) * 0.1).astype(np.float32)
    b = rng.standard_normal(oc).astype(np.float32)
    want = oracle.conv2d(x, wt, b, stride, (pad, pad), groups, extra)
    got = oracle.conv2d(x, wt, b, stride, (pad, pad), groups, extra, fast=True)
    assert got.shape == want.shape
    assert np.array_equal(_bits(got), _bits(want))


@pytest.mark.parametrize("c,oc,k,out_pad,h,w", [
    (128, 128, 3, 1, 9, 13), (64, 8, 3, 1, 5, 31), (192, 128, 4, 0, 7, 11), (20, 3, 3, 1, 4, 5),
    (128, 1, 3, 1, 6, 40),
])
def test_fast_conv_transpose2d_equals_reference_loops_bit_for_bit(cpu_tier, c, oc, k, out_pad, h, w):
    x = rng.standard_normal((c, h, w)).astype(np.float32)
    wt = (rng.standard_normal((c, oc, k, k)) * 0.1).astype(np.float32)
    b = rng.standard_normal(oc).astype(np.float32)
    want = oracle.conv_transpose2d(x, wt, b, 2, 1, out_pad)
    got = oracle.conv_transpose2d(x, wt, b, 2, 1, out_pad, fast=True)
    assert got.shape == want.shape
    assert np.array_equal(_bits(got), _bits(want))


def test_fast_graph_equals_reference_graph():
    """The whole HOP luma + chroma graph on the nn::fast restatement equals the reference-loop
    graph bit for bit (the CPU baseline computes the oracle's result)."""
    import oracle.graphs as og
    from zenjpegai_amd import synth
    py = synth.random_params("hop", "y", seed=12, gain=0.5)
    puv = synth.random_params("hop", "uv", seed=12, gain=0.5)
    y = synth.latent(12, "fg/y", 160, 4, 6)
    uv = synth.latent(12, "fg/uv", 96, 4, 6)
    want = (og.primary(py, "hop", y, 64, 96), og.secondary(puv, "hop", y, uv, 64, 96))
    with og.fast_convs():
        got = (og.primary(py, "hop", y, 64, 96), og.secondary(puv, "hop", y, uv, 64, 96))
    for g, wv in zip(got, want):
        assert np.array_equal(_bits(g), _bits(wv))


# ----------------------------------------------------------------------------- output stage
@pytest.mark.parametrize("name,mode,cases", [("bicubic_align_corners", "bicubic", 6),
                                             ("bilinear_align_corners", "bilinear", 8)])
def test_resize_matches_reference_fixture_exactly(name, mode, cases):
    """The reference's PyTorch vectors (tests/nn_vectors.rs:136-196): exact up-/down-sampling,
    odd sizes, a 4:2:2 width-only case and one-sample axes, bit for bit."""
    t = zjtb.load(name)
    fn = oracle.resize_bicubic if mode == "bicubic" else oracle.resize_bilinear
    for i in range(cases):
        x, want = t[f"x{i}"], t[f"y{i}"]
        got = fn(x, want.shape[1], want.shape[2])
        assert got.tobytes() == want.astype(np.float32).tobytes(), (i, x.shape, want.shape)


def test_resize_closed_forms():
    """Sizes that reduce the resamplers to something known: equal sizes are the identity;
    align_corners keeps the corner samples; a constant plane stays constant (cubic weights sum
    to 1); linear data is reproduced by bilinear (a plausible swapped weight fails this)."""
    rng = np.random.default_rng(5)
    x = rng.uniform(0, 255, (2, 7, 9)).astype(np.float32)
    assert np.array_equal(oracle.resize_bilinear(x, 7, 9), x)
    assert np.array_equal(oracle.resize_bicubic(x, 7, 9), x)
    up = oracle.resize_bicubic(x, 13, 17)
    assert np.array_equal(up[:, [0, 0, -1, -1], [0, -1, 0, -1]], x[:, [0, 0, -1, -1], [0, -1, 0, -1]])
    c = np.full((1, 5, 6), 77.25, np.float32)
    assert np.allclose(oracle.resize_bicubic(c, 9, 11), 77.25, atol=1e-4)
    yy, xx = np.mgrid[0:6, 0:8].astype(np.float32)
    lin = (3 * yy + 2 * xx)[None]
    out = oracle.resize_bilinear(lin, 11, 15)
    oy, ox = np.mgrid[0:11, 0:15].astype(np.float64)
    want = 3 * oy * 5 / 10 + 2 * ox * 7 / 14
    assert np.allclose(out[0], want, atol=1e-4)


def _bt709_yuv(r, g, b):
    """Forward BT.709 (f64): the transform `to_RGB_` inverts, on [0, 255] samples."""
    KR, KG, KB, KBY, KRY = 0.2126, 0.7152, 0.0722, 1.8556, 1.5748
    r, g, b = (np.asarray(a, np.float64) / 255 for a in (r, g, b))
    y = KR * r + KG * g + KB * b
    return y * 255, ((b - y) / KBY + 0.5) * 255, ((r - y) / KRY + 0.5) * 255


def test_yuv_to_rgb_inverts_bt709_and_keeps_gray():
    rng = np.random.default_rng(6)
    rgb = rng.uniform(0, 255, (3, 64, 64))
    y, u, v = _bt709_yuv(*rgb)
    r, g, b = oracle.yuv_to_rgb(y, u, v)
    assert np.abs(np.stack([r, g, b]) - rgb).max() < 2e-3
    # u = v = 127.5 is exactly 0.5 after the range conversion: R = G = B.
    y = rng.uniform(0, 255, (1000,)).astype(np.float32)
    half = np.full_like(y, 127.5)
    r, g, b = oracle.yuv_to_rgb(y, half, half)
    assert np.array_equal(r, g) and np.array_equal(g, b)
    assert np.abs(r - y).max() < 1e-4
    # Out-of-gamut colours clip to [0, 255].
    r, g, b = oracle.yuv_to_rgb(np.float32([255, 0]), np.float32([127.5, 0]), np.float32([255, 127.5]))
    assert r[0] == 255.0 and b[1] == 0.0  # 1 + 1.5748 / 2 and 0 - 1.8556 / 2 clip


def test_quantize_rgb_interleaves_and_rounds_half_even():
    r = np.float32([0.0, 127.5, 255.0, 300.0])
    g = np.float32([255.0, 0.0, 63.75, -1.0])
    b = np.float32([1.0, 2.0, 3.0, 4.0])
    q8 = oracle.quantize_rgb(r, g, b, 8)
    assert q8.shape == (4, 3)
    assert q8[:, 0].tolist() == [0, 128, 255, 255]  # 127.5 -> 128 (even), clamped at 255
    assert q8[:, 1].tolist() == [255, 0, 64, 0]
    q10 = oracle.quantize_rgb(r, g, b, 10)
    assert q10[:, 0].tolist() == [0, 512, 1023, 1023]  # 0.5 * 1023 = 511.5 -> 512
    x = np.linspace(0, 255, 4097, dtype=np.float32)
    q = oracle.quantize_rgb(x, x, x, 10)[:, 0].astype(int)
    assert (np.diff(q) >= 0).all() and q[0] == 0 and q[-1] == 1023


def test_picture_rgb_upsamples_chroma_to_luma_size():
    rng = np.random.default_rng(7)
    y = rng.uniform(0, 255, (9, 13)).astype(np.float32)
    u = rng.uniform(0, 255, (5, 7)).astype(np.float32)
    v = rng.uniform(0, 255, (5, 7)).astype(np.float32)
    q, planes = oracle.picture_rgb(y, u, v, 10)
    uu = oracle.resize_bicubic(u[None], 9, 13)[0]
    vv = oracle.resize_bicubic(v[None], 9, 13)[0]
    want = np.stack(oracle.yuv_to_rgb(y, uu, vv))
    assert np.array_equal(planes, want) and q.shape == (9, 13, 3)
