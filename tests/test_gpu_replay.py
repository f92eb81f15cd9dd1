"""GPU: replay mode (``zjai_picture_set_replay``) -- a picture's whole launch sequence captured once
as a HIP graph and launched again on later runs, as the reference's GPU backend replays its
per-tile dispatch plan (gpu/src/synthesis.rs:1163-1185) -- gives the eager run's bytes on every
replay. Between the replays the same context runs eager work (a conv layer whose tensors come
from the same pools the graph's buffers were taken from), new latents are uploaded and the host
synchronises; each replay is checked against the eager run of the latents it read. The capture
holds no memset or copy, only kernels and fork / join event dependencies.
"""

import numpy as np
import pytest

from zenjpegai_amd import _lib, model, nn, synth

pytestmark = pytest.mark.gpu


def _picture(eng, op, lanes, seed=5):
    """HOP Y + UV (2 x 2 independent regions, two tile shapes, 10-bit 4:2:0) or SOP luma
    untiled (8-bit), He x 0.5 weights."""
    if op == "hop":
        h, w, lh, lw = 256, 320, 16, 20
        tiles = model.synthesis_tiles(h, w, lh, lw, (128, 32), (2, 2))
        sec = model.SynthesisSecondary.load(synth.random_params(op, "uv", seed=seed, gain=0.5), op, eng)
        sv = sh = 2
        bits = 10
    else:
        h, w, lh, lw = 192, 256, 12, 16
        tiles = model.synthesis_tiles(h, w, lh, lw, None)
        sec = None
        sv = sh = 1
        bits = 8
    prim = model.SynthesisPrimary.load(synth.random_params(op, "y", seed=seed, gain=0.5), op, eng)
    pic = model.Picture(eng, prim, sec, lh, lw, h, w, tiles, sv, sh, bit_depth=bits, lanes=lanes)
    return pic, (prim, sec), (lh, lw)


def _latents(seed, lh, lw, uv):
    y = synth.latent(seed, "replay/y", 160, lh, lw)
    return y, (synth.latent(seed, "replay/uv", 96, lh, lw) if uv else None)


def _same(got, want):
    return all((g is None and w is None) or np.array_equal(g, w) for g, w in zip(got, want))


@pytest.mark.parametrize("prec", ["f32", "bf16"])
@pytest.mark.parametrize("op,lanes", [("hop", 1), ("hop", 3), ("sop", 1)])
def test_replayed_picture_equals_eager_runs(prec, op, lanes):
    eng = nn.Engine(0, prec)
    pic, keep, (lh, lw) = _picture(eng, op, lanes)
    lat = [_latents(s, lh, lw, op == "hop") for s in (5, 6)]
    want = []
    for y, uv in lat:
        pic.upload(y, uv)
        before = eng.stats()["kernel_launches"]
        pic.run()
        per_run = eng.stats()["kernel_launches"] - before
        want.append(pic.download())
    assert not _same(want[0], want[1])  # the two latents give different pictures

    rng = np.random.default_rng(7)
    layer = nn.ConvLayer(nn.Conv2d(16, 16, (3, 3), 1, (1, 1), 1,
                                   (0.1 * rng.standard_normal((16, 16, 3, 3))).astype(np.float32)), eng)
    xs = (0.5 * rng.standard_normal((16, 20, 24))).astype(np.float32)
    layer_want = layer.forward(eng, nn.BTensor.from_planar(eng, xs)).to_planar()

    pic.set_replay(True)
    for k in range(5):
        y, uv = lat[k % 2]
        pic.upload(y, uv)
        before = eng.stats()["kernel_launches"]
        pic.run()  # k = 0 captures, then launches the graph
        assert eng.stats()["kernel_launches"] - before == per_run, k
        assert _same(pic.download(), want[k % 2]), f"replay {k}"
        # Eager work on the same context between replays, then a synchronisation.
        out = layer.forward(eng, nn.BTensor.from_planar(eng, xs)).to_planar()
        assert np.array_equal(out, layer_want), k
        eng.sync()
    if lanes > 1:
        pic.set_lanes(2)  # a new lane count captures again
        for k in range(2):
            pic.upload(*lat[k])
            pic.run()
            assert _same(pic.download(), want[k]), f"2 lanes, replay {k}"
        pic.set_lanes(lanes)
    pic.set_replay(False)  # back to eager runs
    pic.upload(*lat[0])
    pic.run()
    assert _same(pic.download(), want[0])
    eng.close()


def test_replay_refuses_capture_while_profiling():
    eng = nn.Engine(0, "f32")
    pic, keep, (lh, lw) = _picture(eng, "sop", 1)
    pic.upload(*_latents(5, lh, lw, False))
    pic.run()
    want = pic.download()
    pic.set_replay(True)
    eng.profile_begin()
    with pytest.raises(nn.HipError):
        pic.run()
    eng.profile_end()
    pic.run()
    assert _same(pic.download(), want)
    eng.close()


@pytest.mark.parametrize("lanes", [1, 3])
def test_a_failure_during_the_capture_leaves_the_picture_usable(lanes):
    """An injected launch failure (host side, before the launch is queued) part way through the
    capture: the run reports the device error, the capture is abandoned with every lane joined
    back and nothing launched, and the next run captures again and replays the eager bytes; an
    eager run afterwards gives them too. (Injected launch failures count the launches issued from
    the host -- eager runs and captures; a replay is one graph launch.)"""
    eng = nn.Engine(0, "f32")
    pic, keep, (lh, lw) = _picture(eng, "hop", lanes)
    pic.upload(*_latents(5, lh, lw, True))
    before = eng.stats()["kernel_launches"]
    pic.run()
    per_run = eng.stats()["kernel_launches"] - before
    want = pic.download()
    for after in (0, per_run // 2):
        pic.set_replay(False)  # drops any graph, so the next run captures
        pic.set_replay(True)
        eng.inject_failure(_lib.FAIL_LAUNCH, after)
        with pytest.raises(nn.HipError) as e:
            pic.run()
        assert e.value.kind == "Device" and "injected launch failure" in str(e.value)
        pic.run()  # captures again (the plan disarmed itself), then replays
        assert _same(pic.download(), want), after
        pic.run()  # a replay of the graph just captured
        assert _same(pic.download(), want), after
    pic.set_replay(False)
    pic.run()
    assert _same(pic.download(), want)
    eng.close()
