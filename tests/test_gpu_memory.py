"""GPU: the device memory estimate of a picture bounds the memory it takes, and admission refuses
a picture over the context's limit before allocating anything.

The reference sizes a decode before it runs (``estimate_memory``, src/decoder/limits.rs:164-245)
and refuses one whose estimate exceeds ``max_memory_bytes`` (``check_header``, :106-111); its own
test asserts that the estimate covers the measured peak of every reference stream
(tests/memory_ref.rs). Here the measured figures are the buffer pools' (``zjai_get_stats``
after ``zjai_release_buffers``): ``pool_peak`` must not exceed the estimate's ``live_bytes`` and
``pool_cached`` not its ``pool_bytes``, on shapes the model was not calibrated on (sizes that are
not multiples of 16, other tilings, f16, two and three lanes, float planes), and neither figure
may be loose by more than 1.6x (+ 2 MiB for the size rounding of tiny tiles).
"""

import numpy as np
import pytest

from zenjpegai_amd import _lib, model, nn, synth

pytestmark = pytest.mark.gpu

# op, precision, height, width, tiling, chroma net, lanes, bit depth
CASES = [
    ("sop", "f16", 200, 312, None, True, 1, 0),
    ("sop", "f32", 1000, 1500, (512, 48), True, 2, 8),
    ("bop", "bf16", 720, 1280, (256, 32), True, 2, 10),
    ("bop", "f32", 600, 904, (512, 64), False, 1, 8),
    ("hop", "f32", 384, 640, (256, 32), True, 3, 10),
    ("hop", "bf16", 720, 1280, (512, 64), True, 1, 0),
]

_NETS = {}


def _engine_and_nets(op, prec):
    key = (op, prec)
    if key not in _NETS:
        eng = nn.Engine(0, prec)
        prim = model.SynthesisPrimary.load(synth.random_params(op, "y", seed=5, gain=0.5), op, eng)
        sec = model.SynthesisSecondary.load(synth.random_params(op, "uv", seed=5, gain=0.5), op, eng)
        _NETS[key] = (eng, prim, sec)
    return _NETS[key]


def _geometry(h, w, tiling):
    lh, lw = -(-h // 16), -(-w // 16)
    return lh, lw, model.synthesis_tiles(h, w, lh, lw, tiling)


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}-{c[1]}-{c[2]}x{c[3]}-L{c[6]}")
def test_estimate_bounds_the_measured_pool_use(case):
    op, prec, h, w, tiling, uv, lanes, bits = case
    print(f"memory estimate case {case}", flush=True)
    eng, prim, sec = _engine_and_nets(op, prec)
    lh, lw, tiles = _geometry(h, w, tiling)
    s = 2 if uv else 1
    est = model.estimate_picture_memory(op, prec, uv, lh, lw, h, w, tiles, s, s, bit_depth=bits,
                                        lanes=lanes)
    eng.release_buffers()
    pic = model.Picture(eng, prim, sec if uv else None, lh, lw, h, w, tiles, s, s, bit_depth=bits,
                        lanes=lanes)
    pic.upload(synth.latent(5, "mem/y", 160, lh, lw), synth.latent(5, "mem/uv", 96, lh, lw) if uv else None)
    pic.run()
    eng.sync()
    st = eng.stats()
    peak, cached = st["pool_peak"], st["pool_cached"]
    assert 0 < peak <= est["live_bytes"] <= 1.6 * peak + (2 << 20), (peak, est)
    assert peak <= cached <= est["pool_bytes"] <= 1.6 * cached + (2 << 20), (cached, est)
    del pic


def test_admission_refuses_a_picture_over_the_limit_before_allocating():
    eng, prim, sec = _engine_and_nets("bop", "bf16")
    h, w = 720, 1280
    lh, lw, tiles = _geometry(h, w, (256, 32))
    nets = prim.device_bytes() + sec.device_bytes()
    assert nets > 0

    def need(lanes):
        e = model.estimate_picture_memory("bop", "bf16", True, lh, lw, h, w, tiles, 2, 2, bit_depth=10,
                                          lanes=lanes)
        return nets + e["picture_bytes"] + e["live_bytes"]

    assert need(4) > need(1)
    eng.release_buffers()
    before = eng.stats()
    try:
        eng.set_memory_limit(need(1) - 1)
        with pytest.raises(_lib.HipError) as ei:
            model.Picture(eng, prim, sec, lh, lw, h, w, tiles, 2, 2, bit_depth=10)
        assert ei.value.code == _lib.E_LIMIT
        assert "exceeds the context's limit" in str(ei.value)
        after = eng.stats()
        assert after["pool_cached"] == before["pool_cached"] and after["kernel_launches"] == before["kernel_launches"]

        # At the limit the picture is admitted on one lane; four lanes need more and are refused,
        # leaving the picture on one lane and usable.
        eng.set_memory_limit(need(1))
        pic = model.Picture(eng, prim, sec, lh, lw, h, w, tiles, 2, 2, bit_depth=10)
        with pytest.raises(_lib.HipError) as ei:
            pic.set_lanes(4)
        assert ei.value.code == _lib.E_LIMIT and pic.lanes == 1
        pic.upload(synth.latent(6, "adm/y", 160, lh, lw), synth.latent(6, "adm/uv", 96, lh, lw))
        pic.run()
        y1, u1, v1 = pic.download()

        # Without a limit the same picture runs on four lanes and gives the same bytes.
        eng.set_memory_limit(0)
        pic.set_lanes(4)
        pic.run()
        y4, u4, v4 = pic.download()
        assert np.array_equal(y1, y4) and np.array_equal(u1, u4) and np.array_equal(v1, v4)
    finally:
        eng.set_memory_limit(0)


def test_net_device_bytes_cover_the_packed_weights():
    """A 16-bit net holds at least half the f32 weight count's bytes (packed 16-bit weights, f32
    biases and vectors) and the f32 net at least the f32 weight bytes."""
    params = synth.random_params("sop", "y", seed=5)
    n_weights = sum(int(np.prod(v.shape)) for v in params.values())
    for prec, per in (("f32", 4), ("bf16", 2)):
        eng = nn.Engine(0, prec)
        net = model.SynthesisPrimary.load(params, "sop", eng)
        assert net.device_bytes() >= per * n_weights
        del net
        eng.close()
