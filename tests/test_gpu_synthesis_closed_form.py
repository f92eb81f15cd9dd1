"""GPU: the HIP synthesis graphs (``graph.hip`` through ``zjai_primary_forward`` /
``zjai_secondary_forward`` / ``zjai_picture_run``) meet the index-map closed forms of
``synthesis_closed_form`` bit for bit -- the same closed forms the CPU oracle is pinned to in
``test_synthesis_oracle.py``. Every convolution output is a single exact product there, so any
summation order gives the same float: equality is the bar, in f32 for the three weight
families and in f16 / bf16 for the integer-valued one (whose activations are exact in 16 bits).

The picture tests run the window-independent family through the tiled picture driver (latent
windows, tile batches, core offsets, chroma decimation, quantisation), up to BASELINE config 5's
own geometry: 3840 x 2160, 2 x 3 independent regions, tile 640 / overlap 128 (24 tiles of four
shapes in batches of 6), 4 lanes, 10-bit 4:2:0 output.
Reference: src/model/synthesis.rs, src/model/attention.rs, src/tools/tiles.rs:127-216,
src/decoder/reconstruct.rs:379-464, src/decoder/output.rs:325-342."""

import numpy as np
import pytest

import oracle
import synthesis_closed_form as cf
from zenjpegai_amd import model, nn, synth

pytestmark = pytest.mark.gpu

BORDER = cf.Family(border=True, gates=True)
LOCAL = cf.Family(border=False, gates=True)
PLAIN = cf.Family(border=True, gates=False)
LOCAL_PLAIN = cf.Family(border=False, gates=False)
FAMILIES = {"border": BORDER, "local": LOCAL, "plain": PLAIN}


def _ceil(a, b):
    return -(-a // b)


@pytest.fixture(scope="module")
def engines():
    e = {p: nn.Engine(0, p) for p in ("f32", "f16", "bf16")}
    yield e
    for v in e.values():
        v.close()


def _lat(seed, h, w):
    lh, lw = _ceil(h, 16), _ceil(w, 16)
    return synth.latent(seed, "gcf/y", 160, lh, lw), synth.latent(seed, "gcf/uv", 96, lh, lw)


def _check_equal(got, want, what):
    assert got.shape == want.shape, (what, got.shape, want.shape)
    d = got != want
    assert not d.any(), (what, int(d.sum()), d.size, np.argwhere(d)[:4].tolist())


CASES = [(op, fam, prec, h, w)
         for op in ("sop", "bop", "hop")
         for fam, precs in (("border", ("f32",)), ("local", ("f32",)), ("plain", ("f32", "f16", "bf16")))
         for prec in precs
         for h, w in ((66, 98), (64, 96))]


@pytest.mark.parametrize("op,fam,prec,h,w", CASES)
def test_primary_is_the_closed_form(engines, op, fam, prec, h, w):
    eng = engines[prec]
    y, _ = _lat(11, h, w)
    f = cf.fit_shift(op, "y", FAMILIES[fam], y, h=h, w=w)
    want = cf.primary(op, f, y, h, w)
    net = model.SynthesisPrimary.load(cf.params(op, "y", f), op, eng)
    got = net.forward(eng, nn.BTensor.from_planar(eng, y), h, w)
    _check_equal(got, want, (op, fam, prec, h, w))


@pytest.mark.parametrize("op,fam,prec,h,w", CASES)
def test_secondary_is_the_closed_form(engines, op, fam, prec, h, w):
    eng = engines[prec]
    y, uv = _lat(12, h, w)
    f = cf.fit_shift(op, "uv", FAMILIES[fam], y, uv, h=h, w=w)
    want = cf.secondary(op, f, y, uv, h, w)
    net = model.SynthesisSecondary.load(cf.params(op, "uv", f), op, eng)
    got = net.forward(eng, nn.BTensor.from_planar(eng, y), nn.BTensor.from_planar(eng, uv), h, w)
    _check_equal(got, want, (op, fam, prec, h, w))


def _shift_for(v):
    m, s = float(np.max(np.abs(v))), 0
    while m * 2.0 ** -s * 128 >= 127:
        s += 1
    return s


def _local_picture_case(op, fam, h, w, seed, sv, sh):
    """Weights, latents and the closed-form planes. The output shift only scales the last
    layer's single product by a power of two (exact), so the planes of the shifted nets are
    denormalize(2^-s x the unshifted pre-denormalize planes)."""
    lh, lw = _ceil(h, 16), _ceil(w, 16)
    y = synth.latent(seed, "gpic/y", 160, lh, lw)
    uv = synth.latent(seed, "gpic/uv", 96, lh, lw)
    ry, ru, rv = cf.local_picture(op, fam, fam, y, uv, h, w, sv, sh, denorm=False)
    sy, su = _shift_for(ry), _shift_for(np.stack([ru, rv]))
    want = [oracle.denormalize(ry * np.float32(2.0 ** -sy)),
            oracle.denormalize(ru * np.float32(2.0 ** -su)),
            oracle.denormalize(rv * np.float32(2.0 ** -su))]
    return fam.with_shift(sy), fam.with_shift(su), y, uv, want


def _run_picture(eng, op, fy, fu, y, uv, h, w, tiling, regions, sv, sh, bits, lanes):
    tiles = model.synthesis_tiles(h, w, y.shape[1], y.shape[2], tiling, regions)
    prim = model.SynthesisPrimary.load(cf.params(op, "y", fy), op, eng)
    sec = model.SynthesisSecondary.load(cf.params(op, "uv", fu), op, eng)
    return tiles, model.synthesize(eng, prim, sec, y, uv, h, w, tiles, sv, sh, bit_depth=bits,
                                   lanes=lanes)


@pytest.mark.parametrize("op,h,w,tiling,regions,sv,sh", [
    ("sop", 256, 384, (128, 32), None, 2, 2),
    ("bop", 200, 296, (128, 64), None, 2, 1),
    ("hop", 256, 512, (128, 64), (1, 2), 2, 2),
    ("hop", 232, 344, (96, 32), (2, 2), 1, 1),
])
@pytest.mark.parametrize("bits", [0, 10])
def test_tiled_picture_is_the_local_closed_form(engines, op, h, w, tiling, regions, sv, sh, bits):
    """Float planes bit for bit; 10-bit planes equal quantize_plane of the closed form."""
    fy, fu, y, uv, want = _local_picture_case(op, LOCAL, h, w, 13, sv, sh)
    assert np.array_equal(want[0], cf.local_picture(op, fy, fu, y, uv, h, w, sv, sh)[0])
    tiles, got = _run_picture(engines["f32"], op, fy, fu, y, uv, h, w, tiling, regions, sv, sh,
                              bits, lanes=2)
    assert len(tiles) > 1
    for g, wv, name in zip(got, want, "yuv"):
        _check_equal(g, oracle.quantize_plane(wv, bits) if bits else wv, (op, name, bits))


@pytest.mark.parametrize("prec,fam", [("f32", "local"), ("bf16", "local_plain")])
def test_config5_geometry_is_the_local_closed_form(engines, prec, fam):
    """BASELINE config 5 exactly as bench.py builds it -- 3840 x 2160, latents 135 x 240, 2 x 3
    independent regions, tile 640 / overlap 128, 10-bit 4:2:0, 4 lanes -- with window-independent
    index-map weights: the 10-bit planes equal quantize_plane of the closed form, every sample."""
    h, w, op = 2160, 3840, "hop"
    f = LOCAL if fam == "local" else LOCAL_PLAIN
    fy, fu, y, uv, want = _local_picture_case(op, f, h, w, 14, 2, 2)
    tiles, got = _run_picture(engines[prec], op, fy, fu, y, uv, h, w, (640, 128), (2, 3), 2, 2, 10,
                              lanes=4)
    assert len(tiles) == 24
    assert len({(t.image.width, t.image.height) for t in tiles}) == 4
    print(f"config-5 geometry {prec}: {len(tiles)} tiles, distinct 10-bit luma values "
          f"{len(np.unique(got[0]))}")
    for g, wv, name in zip(got, want, "yuv"):
        _check_equal(g, oracle.quantize_plane(wv, 10), (prec, name))
