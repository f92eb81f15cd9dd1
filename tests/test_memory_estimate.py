"""CPU: the device memory estimate of a picture (``zjai_picture_estimate_memory``, the
counterpart of the reference's ``estimate_memory``, src/decoder/limits.rs:164-245).

* It bounds the pool use measured on an MI355X (``tests/golden/pool_use_mi355x.json``, written
  by ``tests/golden/pool_use.py``): for every measured picture ``pool_peak <= live_bytes`` and
  ``pool_cached <= pool_bytes``, each within 1.6x (+ 2 MiB), as the reference's test holds its
  estimate to cover every measured stream (tests/memory_ref.rs).
* ``picture_bytes`` is the latents (160 + 96 f32 planes of the latent size) and the output planes
  (2 bytes per sample at 8-16 bits, 4 as float planes; chroma subsampled).
* Lanes run their batches at once: the live figure grows with the lane count up to the number of
  batches and stays there; the pools' figure does not depend on it when every batch has its own
  shape.
* Invalid arguments are refused as zjai_picture_create refuses them.
"""

import json
import os

import pytest

from zenjpegai_amd import _lib, model

FIXTURE = os.path.join(os.path.dirname(__file__), "golden", "pool_use_mi355x.json")


def _est(op, prec, uv, h, w, tiling=None, regions=None, lanes=1, bits=10, out=None):
    lh, lw = -(-h // 16), -(-w // 16)
    tiles = model.synthesis_tiles(h, w, lh, lw, tiling, regions)
    s = 2 if uv else 1
    oh, ow = out if out else (h, w)
    return model.estimate_picture_memory(op, prec, uv, lh, lw, h, w, tiles, s, s, oh, ow, bits, lanes), tiles


def _cases():
    with open(FIXTURE) as f:
        return json.load(f)


@pytest.mark.parametrize("rec", _cases(), ids=lambda r: "{op}-{precision}-{height}x{width}-uv{uv}-L{lanes}".format(**r))
def test_estimate_bounds_measured_pool_use(rec):
    e, _ = _est(rec["op"], rec["precision"], rec["uv"], rec["height"], rec["width"],
                tuple(rec["tiling"]) if rec["tiling"] else None,
                tuple(rec["regions"]) if rec["regions"] else None, rec["lanes"])
    peak, cached = rec["pool_peak"], rec["pool_cached"]
    assert peak <= e["live_bytes"] <= 1.6 * peak + (2 << 20)
    assert cached <= e["pool_bytes"] <= 1.6 * cached + (2 << 20)


def test_fixture_covers_every_operating_point_and_storage_size():
    seen = {(r["op"], r["precision"], r["uv"]) for r in _cases()}
    for op in ("sop", "bop", "hop"):
        for prec in ("f32", "bf16"):
            assert (op, prec, True) in seen and (op, prec, False) in seen


@pytest.mark.parametrize("uv,bits,sub", [(True, 10, 2), (True, 0, 1), (False, 8, 1), (False, 0, 1)])
def test_picture_bytes_are_the_latents_and_planes(uv, bits, sub):
    h, w = 1000, 1500
    lh, lw = -(-h // 16), -(-w // 16)
    tiles = model.synthesis_tiles(h, w, lh, lw, (512, 64))
    e = model.estimate_picture_memory("sop", "f32", uv, lh, lw, h, w, tiles, sub, sub, 997, 1499, bits, 1)
    sample = 2 if bits else 4
    want = 4 * 160 * lh * lw + sample * 997 * 1499
    if uv:
        want += 4 * 96 * lh * lw + 2 * sample * (-(-997 // sub)) * (-(-1499 // sub))
    assert e["picture_bytes"] == want


def test_live_grows_with_lanes_up_to_the_batch_count():
    h, w = 2160, 3840  # four tile shapes, one batch of six tiles each
    e = [_est("hop", "f32", True, h, w, (640, 128), (2, 3), lanes=n)[0] for n in (1, 2, 4, 8)]
    assert e[0]["live_bytes"] < e[1]["live_bytes"] < e[2]["live_bytes"] == e[3]["live_bytes"]
    assert e[0]["pool_bytes"] == e[2]["pool_bytes"] == e[3]["pool_bytes"]
    for x in e:
        assert x["live_bytes"] <= x["pool_bytes"]
    # 16-bit storage halves the activations, give or take the f32 scratch of a few kernels.
    b = _est("hop", "bf16", True, h, w, (640, 128), (2, 3), lanes=4)[0]
    assert 0.45 < b["live_bytes"] / e[2]["live_bytes"] < 0.56


def test_working_set_scales_with_the_tile_area():
    small = _est("bop", "f32", False, 512, 512)[0]
    big = _est("bop", "f32", False, 1024, 1024)[0]
    grow = (big["live_bytes"] - small["live_bytes"]) / (1024 * 1024 - 512 * 512)
    assert 45 < grow < 60  # bytes per sample of a BOP f32 batch item, measured 50.5


@pytest.mark.parametrize("bad", [
    dict(op=3), dict(prec=7), dict(lanes=0), dict(lanes=9), dict(sub=3), dict(bits=7),
    dict(out=(1100, 1000)), dict(uv=2),
])
def test_invalid_arguments_are_refused(bad):
    h, w = 1024, 1024
    lh, lw = 64, 64
    tiles = model._tile_array(model.synthesis_tiles(h, w, lh, lw, None))
    e = _lib.ZjaiMemoryEstimate()
    oh, ow = bad.get("out", (h, w))
    sub = bad.get("sub", 1)
    rc = _lib.lib().zjai_picture_estimate_memory(
        bad.get("op", 0), bad.get("prec", 0), bad.get("uv", 1), lh, lw, h, w, tiles, len(tiles), sub, sub,
        oh, ow, bad.get("bits", 10), bad.get("lanes", 1), e)
    assert rc == _lib.E_INVALID_ARGUMENT
