"""CPU pins of the analysis-transform oracle (src/model/analysis.rs): the padding rule, replicate
padding and feature clipping against brute force and the reference's own unit tests
(src/model/load.rs:121-170), and the whole BOP graph against a closed form: with index-map
weights (each stride-2 conv copies input channel k at its bottom-right tap to output channel k,
every ResAU's 1x1 is zero so its gate is the identity) the latent is the normalised picture
sampled at composed, clamped indices -- which a zero pad, a wrong pad side or a wrong stride
would break."""

import numpy as np
import pytest

import oracle.graphs as og
from zenjpegai_amd import synth


def _ceil(a, b):
    return -(-a // b)


def test_pad_amount_is_one_exactly_when_the_map_is_odd():
    for d in (1, 2, 4, 8):
        for n in range(1, 300):
            assert og.pad_amount(n, d) == _ceil(n, d) % 2, (n, d)


def test_replicate_pad_copies_the_last_row_and_column():
    x = np.arange(2 * 3 * 4, dtype=np.float32).reshape(2, 3, 4)
    y = og.replicate_pad(x, 2, 1)
    assert y.shape == (2, 5, 5)
    for c in range(2):
        for i in range(5):
            for j in range(5):
                assert y[c, i, j] == x[c, min(i, 2), min(j, 3)]
    assert og.replicate_pad(x, 0, 0) is x


def test_clip_channels_matches_the_reference_unit_tests():
    """src/model/load.rs:129-170: per-channel clamps; lists shorter than the channel count leave
    the tail alone; NaN stays NaN (f32::clamp)."""
    x = np.stack([np.full((2, 3), c * 10.0, np.float32) for c in range(10)])
    y = og.clip_channels(x, [20.0] * 10, [70.0] * 10)
    for c in range(10):
        assert np.all(y[c] == np.clip(c * 10.0, 20.0, 70.0))
    y = og.clip_channels(x, [20.0] * 4, [70.0] * 6)
    assert np.all(y[:4] == np.clip(x[:4], 20, 70)) and np.array_equal(y[4:], x[4:])
    z = og.clip_channels(np.array([[[np.nan, -5.0, 5.0]]], np.float32), [0.0], [1.0])
    assert np.isnan(z[0, 0, 0]) and z[0, 0, 1] == 0.0 and z[0, 0, 2] == 1.0


def test_normalize_is_exact():
    x = np.arange(256, dtype=np.float32)[None, None, :]
    assert np.array_equal(og.normalize(x), ((x.astype(np.float64) - 127.5) / 128.0).astype(np.float32))


def index_map_params(op, component):
    """BOP analysis weights whose graph is an index map (the docstring above)."""
    p = synth.random_analysis_params(op, component, seed=7)
    for name in p:
        if name.endswith(".bias"):
            p[name] = np.zeros_like(p[name])
    for name in ("conv1", "conv2", "conv3", "conv4"):
        if f"{name}.weight" not in p:
            continue
        w = np.zeros_like(p[f"{name}.weight"])
        for k in range(min(w.shape[0], w.shape[1])):
            w[k, k, 2, 2] = 1.0
        p[f"{name}.weight"] = w
    for a in ("act1", "act2", "act3"):
        p[f"{a}.conv2.weight"] = np.zeros_like(p[f"{a}.conv2.weight"])
    w5 = np.zeros_like(p["conv5.weight"])
    for k in range(min(w5.shape[0], w5.shape[1])):
        w5[k, k, 0, 0] = 1.0
    p["conv5.weight"] = w5
    return p


def index_map_closed_form(x, stages):
    """normalize(x)[k] sampled at r(i), c(j): each stride-2 bottom-right tap reads input row
    2i + 1 of a map padded by replicating its last row, i.e. min(2i + 1, rows - 1)."""
    c, h, w = x.shape
    n = og.normalize(x)
    rows, cols = np.arange(_ceil(h, 2 ** stages)), np.arange(_ceil(w, 2 ** stages))
    for s in range(stages, 0, -1):
        rows = np.minimum(2 * rows + 1, _ceil(h, 2 ** (s - 1)) - 1)
        cols = np.minimum(2 * cols + 1, _ceil(w, 2 ** (s - 1)) - 1)
    return n[:, rows][:, :, cols]


@pytest.mark.parametrize("component,h,w", [("y", 64, 64), ("y", 70, 90), ("y", 33, 47),
                                           ("uv", 40, 24), ("uv", 21, 35)])
def test_bop_analysis_index_map_closed_form(component, h, w):
    p = index_map_params("bop", component)
    c = 1 if component == "y" else 12
    x = synth.picture(8, f"im{component}", c, h, w)
    if component == "y":
        got, stages = og.analysis_primary(p, "bop", x), 4
    else:
        got, stages = og.analysis_secondary(p, "bop", x), 3
    want = index_map_closed_form(x, stages)
    assert got.shape == ((160 if component == "y" else 96),) + want.shape[1:]
    assert np.array_equal(got[:c], want)
    assert not np.any(got[c:])


def test_shapes_and_the_sop_refusal():
    for op in ("bop", "hop"):
        p = synth.random_analysis_params(op, "y", seed=1, gain=0.5)
        assert og.analysis_primary(p, op, synth.picture(1, "s", 1, 50, 70)).shape == (160, 4, 5)
        q = synth.random_analysis_params(op, "uv", seed=1, gain=0.5)
        assert og.analysis_secondary(q, op, synth.picture(1, "s", 12, 50, 70)).shape == (96, 7, 9)
    with pytest.raises(ValueError):
        og.analysis_primary(p, "sop", synth.picture(1, "s", 1, 16, 16))


def test_clip_lists_apply_only_when_asked():
    p = synth.random_analysis_params("bop", "uv", seed=2, gain=0.5)
    x = synth.picture(2, "clip", 12, 32, 32)
    plain = og.analysis_secondary(p, "bop", x)
    p["clip_thres.E5B.MinList"] = np.full(50, -0.01, np.float32)
    p["clip_thres.E5B.MaxList"] = np.full(60, 0.01, np.float32)
    assert np.array_equal(og.analysis_secondary(p, "bop", x), plain)
    clipped = og.analysis_secondary(p, "bop", x, clip=True)
    assert np.array_equal(clipped[:50], np.clip(plain[:50], -0.01, 0.01))
    assert np.array_equal(clipped[50:], plain[50:])
