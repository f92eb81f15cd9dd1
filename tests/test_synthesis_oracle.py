"""CPU pins of the synthesis-graph oracle (``oracle/graphs.py``: light / HOP primary, secondary,
residual block, ResAU, CAB, transformer block, TAM, upsample, ``synthesize``) against index-map
closed forms (``synthesis_closed_form``): with single-tap power-of-two weights each net is an
explicit composition of shifts, samplings, up-samplings, crops and pixel shuffles of the latent,
evaluated with numpy index arithmetic, never a convolution. Sizes are chosen so that every crop
of the graph (``ceil(h / 8)``, ``/ 4``, ``/ 2``) removes a row and a column; the border family
shows the zero padding of every map edge in the output, so a crop of the wrong size or at the
wrong place changes samples.

The second half plants plausible wiring mistakes in the oracle (monkeypatched copies of its
functions, CPU only) and checks that the closed forms catch each one: a crop at /4 instead of
/8, a dropped crop, a swapped ``cat`` order, CAB's mask fed from the trunk, TAM's down/up-sampling
on the chroma net or missing on the luma net, a residual skip from the wrong tensor, a transposed
pixel shuffle.

Reference: src/model/synthesis.rs:356-390 (HopPrimary), :550-580 (LightPrimary), :755-773,
:884-909, :1004-1038 (secondary); src/model/attention.rs:35-43, :119-139, :328-372, :528-545;
src/decoder/reconstruct.rs:379-464 (tile stitching, chroma decimation)."""

import numpy as np
import pytest

import oracle
import oracle.graphs as og
from oracle import geometry as geo
import synthesis_closed_form as cf
from zenjpegai_amd import synth

BORDER = cf.Family(border=True, gates=True)
LOCAL = cf.Family(border=False, gates=True)
PLAIN = cf.Family(border=True, gates=False)
FAMILIES = {"border": BORDER, "local": LOCAL, "plain": PLAIN}

# (h, w): 66 x 98 and 33 x 49 make every crop of the graph remove a row and a column; 64 x 96
# removes none; 70 x 90 some.
SIZES = [(66, 98), (33, 49), (64, 96), (70, 90)]


def _ceil(a, b):
    return -(-a // b)


def _latents(seed, h, w, extra_luma=(0, 0)):
    lh, lw = _ceil(h, 16), _ceil(w, 16)
    y = synth.latent(seed, "cf/y", 160, lh + extra_luma[0], lw + extra_luma[1])
    uv = synth.latent(seed, "cf/uv", 96, lh, lw)
    return y, uv


def _primary_case(op, fam, h, w, seed=3):
    y, _ = _latents(seed, h, w)
    fam = cf.fit_shift(op, "y", fam, y, h=h, w=w)
    return cf.params(op, "y", fam), y, cf.primary(op, fam, y, h, w)


def _secondary_case(op, fam, h, w, seed=4, extra_luma=(0, 0)):
    y, uv = _latents(seed, h, w, extra_luma)
    fam = cf.fit_shift(op, "uv", fam, y, uv, h=h, w=w)
    return cf.params(op, "uv", fam), y, uv, cf.secondary(op, fam, y, uv, h, w)


def test_the_crop_sizes_remove_rows():
    """The sizes above do exercise the crops: ceil(h / 8) < 2 ceil(h / 16) and so on."""
    for h in (66, 98, 33, 49):
        assert _ceil(h, 8) < 2 * _ceil(h, 16)
        assert _ceil(h, 4) < 2 * _ceil(h, 8)
        assert _ceil(h, 2) < 2 * _ceil(h, 4)


@pytest.mark.parametrize("fam", list(FAMILIES))
@pytest.mark.parametrize("op", ["sop", "bop", "hop"])
@pytest.mark.parametrize("h,w", SIZES)
def test_primary_oracle_is_the_closed_form(op, fam, h, w):
    p, y, want = _primary_case(op, FAMILIES[fam], h, w)
    got = og.primary(p, op, y, h, w)
    assert got.shape == want.shape
    assert np.array_equal(got, want)
    # Informative: the planes are not saturated and vary.
    assert 0 < want.min() and want.max() < 255 and len(np.unique(want)) > 5


@pytest.mark.parametrize("fam", list(FAMILIES))
@pytest.mark.parametrize("op", ["sop", "bop", "hop"])
@pytest.mark.parametrize("h,w", SIZES[:2])
def test_secondary_oracle_is_the_closed_form(op, fam, h, w):
    p, y, uv, want = _secondary_case(op, FAMILIES[fam], h, w)
    got = og.secondary(p, op, y, uv, h, w)
    assert got.shape == want.shape
    assert np.array_equal(got, want)
    assert 0 < want.min() and want.max() < 255 and len(np.unique(want)) > 5


@pytest.mark.parametrize("op", ["sop", "hop"])
def test_secondary_crops_a_larger_luma_latent(op):
    """SynthesisSecondary crops both latents to the common size (synthesis.rs:1012-1020)."""
    p, y, uv, want = _secondary_case(op, BORDER, 33, 49, extra_luma=(2, 1))
    assert y.shape[1:] != uv.shape[1:]
    assert np.array_equal(og.secondary(p, op, y, uv, 33, 49), want)


def test_transformer_block_closed_form():
    """One TransformerBlock (attention.rs:328-372) of the border family on a 6 x 10 map: the
    layer norms output their biases, zero queries give uniform attention, and the block adds
    the two depthwise border patterns to x."""
    d = 64
    p = {}
    cf._tab(p, BORDER, "t", d)
    x = synth.laplace(9, "tab", (d, 6, 10), 2.0)
    got = og.transformer_block(p, "t", x)
    assert np.array_equal(got, cf.tab(BORDER, x))
    assert not np.array_equal(got, x)
    attn = oracle.channel_attention(np.zeros((3 * d, 6, 10), np.float32) + 1, 4, np.ones(4, np.float32))
    assert np.all(np.isfinite(attn))


# ----------------------------------------------------------------------- tiled pictures
PICTURES = [
    # op, height, width, tiling, regions, sv, sh
    ("sop", 256, 384, (128, 32), None, 2, 2),
    ("bop", 200, 296, (128, 64), None, 2, 1),
    ("hop", 256, 512, (128, 64), (1, 2), 2, 2),
    ("hop", 232, 344, (96, 32), (2, 2), 1, 1),
]


def picture_case(op, height, width, seed=5):
    lh, lw = _ceil(height, 16), _ceil(width, 16)
    y = synth.latent(seed, "pic/y", 160, lh, lw)
    uv = synth.latent(seed, "pic/uv", 96, lh, lw)
    fy = LOCAL.with_shift(0)
    fu = LOCAL.with_shift(0)
    ry, ru, rv = cf.local_picture(op, fy, fu, y, uv, height, width, denorm=False)
    fy = fy.with_shift(_shift_for(ry))
    fu = fu.with_shift(_shift_for(np.stack([ru, rv])))
    return fy, fu, y, uv


def _shift_for(v):
    m, s = float(np.max(np.abs(v))), 0
    while m * 2.0 ** -s * 128 >= 127:
        s += 1
    return s


@pytest.mark.parametrize("op,height,width,tiling,regions,sv,sh", PICTURES)
def test_tiled_synthesis_is_the_untiled_local_net(op, height, width, tiling, regions, sv, sh):
    """Local family: each output block depends only on its latent column, so the stitched tile
    cores (and the kept chroma rows / columns) equal the closed form of the whole picture; a
    wrong latent window, core offset or decimation phase breaks it."""
    fy, fu, y, uv = picture_case(op, height, width)
    rg = geo.image_region_grid(height, width, *regions) if regions else None
    tiles = geo.synthesis_tiles(height, width, y.shape[1], y.shape[2], tiling, rg)
    assert len(tiles) > 1
    py, puv = cf.params(op, "y", fy), cf.params(op, "uv", fu)
    got = og.synthesize(py, puv, op, y, uv, height, width, tiles, sv, sh)
    want = cf.local_picture(op, fy, fu, y, uv, height, width, sv, sh)
    for g, wv in zip(got, want):
        assert g.shape == wv.shape
        assert np.array_equal(g, wv)
    assert len(np.unique(want[0])) > 50


# ------------------------------------------------------------------ planted mistakes
def _differs(fn, want):
    """True when the (mutated) oracle call raises or disagrees with the closed form."""
    try:
        got = fn()
    except (ValueError, KeyError, AssertionError, oracle.OracleError):
        return True
    return got.shape != want.shape or not np.array_equal(got, want)


def _crop_mutant(index, how):
    """og.crop with the ``index``-th call changed: ``how`` = "skip" (no crop), "quarter" (the
    /8 crop taken at /4: the next power of two), or "eighth" (the /4 crop taken at /8)."""
    real = og.crop
    calls = {"n": 0}

    def crop(x, h, w):
        i = calls["n"]
        calls["n"] += 1
        if i != index:
            return real(x, h, w)
        if how == "skip":
            return x
        if how == "quarter":
            return real(x, 2 * h - 1, 2 * w - 1)
        return real(x, (h + 1) // 2, (w + 1) // 2)

    return crop


@pytest.mark.parametrize("op", ["sop", "hop"])
@pytest.mark.parametrize("index,how", [(0, "skip"), (1, "skip"), (0, "quarter"), (1, "eighth"),
                                       (2, "skip")])
def test_closed_form_catches_a_wrong_crop(monkeypatch, op, index, how):
    if op == "sop" and index == 2:
        pytest.skip("the light nets crop twice")
    p, y, want = _primary_case(op, BORDER, 66, 98)
    monkeypatch.setattr(og, "crop", _crop_mutant(index, how))
    assert _differs(lambda: og.primary(p, op, y, 66, 98), want)


@pytest.mark.parametrize("op", ["sop", "bop", "hop"])
@pytest.mark.parametrize("which", [0, 1])
def test_closed_form_catches_a_swapped_cat(monkeypatch, op, which):
    """``which`` = 0: cat(yUV, yY) before the combine conv; 1: cat(yUV, info) after it."""
    p, y, uv, want = _secondary_case(op, BORDER, 66, 98)

    class SwappedNp:
        def __init__(self):
            self.n = 0

        def __getattr__(self, name):
            return getattr(np, name)

        def concatenate(self, parts, axis=0):
            i = self.n
            self.n += 1
            if i == which:
                parts = list(parts)[::-1]
            return np.concatenate(parts, axis)

    monkeypatch.setattr(og, "np", SwappedNp())
    assert _differs(lambda: og.secondary(p, op, y, uv, 66, 98), want)


def test_closed_form_catches_cab_mask_fed_from_the_trunk(monkeypatch):
    p, y, want = _primary_case("hop", BORDER, 66, 98)

    def cab(p_, pfx, x):
        trunk = og.residual_block(p_, f"{pfx}.residual_trunk.0", x)
        trunk = og.residual_block(p_, f"{pfx}.residual_trunk.1", trunk)
        m = og.conv3x3(p_, f"{pfx}.subscale", trunk, stride=2)  # planted: trunk, not x
        m = og.residual_block(p_, f"{pfx}.residual_mask2.0", m)
        m = og.residual_block(p_, f"{pfx}.residual_mask3.0", m)
        m = og.conv3x3_t(p_, f"{pfx}.upscale", m)
        return og.add(og.mul(trunk, og.sigmoid(m)), x)

    monkeypatch.setattr(og, "cab", cab)
    assert _differs(lambda: og.primary(p, "hop", y, 66, 98), want)


def test_closed_form_catches_cab_skip_from_the_trunk(monkeypatch):
    p, y, want = _primary_case("hop", BORDER, 66, 98)

    def cab(p_, pfx, x):
        trunk = og.residual_block(p_, f"{pfx}.residual_trunk.0", x)
        trunk = og.residual_block(p_, f"{pfx}.residual_trunk.1", trunk)
        m = og.conv3x3(p_, f"{pfx}.subscale", x, stride=2)
        m = og.residual_block(p_, f"{pfx}.residual_mask2.0", m)
        m = og.residual_block(p_, f"{pfx}.residual_mask3.0", m)
        m = og.conv3x3_t(p_, f"{pfx}.upscale", m)
        return og.add(og.mul(trunk, og.sigmoid(m)), trunk)  # planted: + trunk, not + x

    monkeypatch.setattr(og, "cab", cab)
    assert _differs(lambda: og.primary(p, "hop", y, 66, 98), want)


@pytest.mark.parametrize("index", [0, 1])
def test_closed_form_catches_a_dropped_crop_in_bop(monkeypatch, index):
    """BOP at 70 x 90 (h mod 8 = 6: the /4 crop keeps the odd row that reads past the /8 crop)."""
    p, y, want = _primary_case("bop", BORDER, 70, 90)
    monkeypatch.setattr(og, "crop", _crop_mutant(index, "skip"))
    assert _differs(lambda: og.primary(p, "bop", y, 70, 90), want)


@pytest.mark.parametrize("op,index", [("sop", 1), ("bop", 1), ("hop", 1), ("hop", 2), ("hop", 0)])
def test_closed_form_catches_a_dropped_crop_in_the_chroma_net(monkeypatch, op, index):
    """Crop 0 is the luma latent's crop to the chroma size (a larger luma latent here), 1 the
    /8 crop, 2 HOP's /4 crop."""
    p, y, uv, want = _secondary_case(op, BORDER, 66, 98, extra_luma=(1, 1))
    monkeypatch.setattr(og, "crop", _crop_mutant(index, "skip"))
    assert _differs(lambda: og.secondary(p, op, y, uv, 66, 98), want)


def test_closed_form_catches_tam_downsampling_on_the_chroma_net(monkeypatch):
    p, y, uv, want = _secondary_case("hop", BORDER, 66, 98)
    q = {}
    cf._tam(q, BORDER, "TAM", 64, True)
    p = dict(p, **{k: v for k, v in q.items() if "_conv" in k})
    real = og.tam
    monkeypatch.setattr(og, "tam", lambda p_, pfx, x, ds: real(p_, pfx, x, True))
    assert _differs(lambda: og.secondary(p, "hop", y, uv, 66, 98), want)


def test_closed_form_catches_tam_without_downsampling_on_the_luma_net(monkeypatch):
    p, y, want = _primary_case("hop", BORDER, 66, 98)
    real = og.tam
    monkeypatch.setattr(og, "tam", lambda p_, pfx, x, ds: real(p_, pfx, x, False))
    assert _differs(lambda: og.primary(p, "hop", y, 66, 98), want)


def test_closed_form_catches_a_residual_skip_from_the_wrong_tensor(monkeypatch):
    p, y, want = _primary_case("hop", BORDER, 66, 98)

    def residual_block(p_, pfx, x):
        t = og.relu(og.conv3x3(p_, f"{pfx}.conv1", x))
        return og.add(og.conv3x3(p_, f"{pfx}.conv2", t), t)  # planted: + t, not + x

    monkeypatch.setattr(og, "residual_block", residual_block)
    assert _differs(lambda: og.primary(p, "hop", y, 66, 98), want)


def test_closed_form_catches_a_transposed_pixel_shuffle(monkeypatch):
    p, y, want = _primary_case("sop", BORDER, 66, 98)
    real = og.pixel_shuffle

    def pixel_shuffle(x, r):
        out = real(x, r)
        c, h, w = out.shape
        return np.ascontiguousarray(
            out.reshape(c, h // r, r, w // r, r).transpose(0, 1, 4, 3, 2).reshape(c, h, w))

    monkeypatch.setattr(og, "pixel_shuffle", pixel_shuffle)
    assert _differs(lambda: og.primary(p, "sop", y, 66, 98), want)


def test_closed_form_catches_resau_gate_on_the_relu6_input(monkeypatch):
    p, y, want = _primary_case("bop", BORDER, 66, 98)

    def res_au(p_, pfx, x):
        w = p_[f"{pfx}.conv.weight"]
        t = og.conv2d(og.relu6(x), w, None, 1, (1, 1), x.shape[0] // w.shape[1])
        return og.gate(og.relu6(x), og.conv1x1(p_, f"{pfx}.conv2", t))  # planted

    monkeypatch.setattr(og, "res_au", res_au)
    assert _differs(lambda: og.primary(p, "bop", y, 66, 98), want)


def test_closed_form_catches_a_wrong_core_offset(monkeypatch):
    op, height, width = "hop", 256, 512
    fy, fu, y, uv = picture_case(op, height, width)
    tiles = geo.synthesis_tiles(height, width, y.shape[1], y.shape[2], (128, 64),
                                geo.image_region_grid(height, width, 1, 2))
    bad = [geo.SynthesisTile(t.image, t.latent, t.core, (t.core_offset[0] + (i == 1), t.core_offset[1]))
           for i, t in enumerate(tiles)]
    py, puv = cf.params(op, "y", fy), cf.params(op, "uv", fu)
    want = cf.local_picture(op, fy, fu, y, uv, height, width, 2, 2)
    assert _differs(lambda: og.synthesize(py, puv, op, y, uv, height, width, bad, 2, 2)[0], want[0])
