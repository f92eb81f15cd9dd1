"""GPU parity of BASELINE config 5 -- HOP luma + chroma synthesis of a 3840 x 2160 4:2:0 picture,
2 x 3 independent regions, tile 640 / overlap 128 (24 tiles of four shapes, batches of 6), 4
lanes, 10-bit output -- built exactly as bench.py builds it, against the CPU oracle's
``synthesize`` (src/decoder/reconstruct.rs:379-464 over src/model/synthesis.rs) on the same
random-init weights and latents. The oracle runs its convolutions on the nn::fast restatement
(bit-identical to the reference loops; ``test_oracle.py``) so the 24 tiles take ~30 s.

Gates (tests/decode_ref.rs:157-190 for the reference's own):
* He-normal x 0.5 weights (outputs span the range): 8-bit and 10-bit reconstructions differ by
  at most one step in at most 0.05 % of samples.
* The bench's own He-normal weights (gain 1): activations reach ~1e5 before denormalize and
  every sample saturates; samples whose value is a small difference of large terms flip between
  the clamp edges under any change of summation order -- the oracle against itself with every
  weight moved by one ulp does the same (``test_conditioning.py``). The 10-bit planes are held
  to the 0.05 % fraction bound, or -- on the chroma planes, where the oracle's own spread under
  that perturbation is ~0.09 % -- to at most 3x that spread; the step statistics are printed.
"""

import numpy as np
import pytest

import oracle
import oracle.graphs as og
from oracle import geometry as geo
from zenjpegai_amd import model, nn, synth

pytestmark = pytest.mark.gpu

H, W, LH, LW = 2160, 3840, 135, 240


def _workload(seed, gain):
    py = synth.random_params("hop", "y", seed=seed, gain=gain)
    puv = synth.random_params("hop", "uv", seed=seed, gain=gain)
    y = synth.latent(seed, "cfg5/y", 160, LH, LW)
    uv = synth.latent(seed, "cfg5/uv", 96, LH, LW)
    return py, puv, y, uv


def _gpu(eng, py, puv, y, uv, bits):
    tiles = model.synthesis_tiles(H, W, LH, LW, (640, 128), (2, 3))
    assert len(tiles) == 24
    prim = model.SynthesisPrimary.load(py, "hop", eng)
    sec = model.SynthesisSecondary.load(puv, "hop", eng)
    return model.synthesize(eng, prim, sec, y, uv, H, W, tiles, 2, 2, bit_depth=bits, lanes=4)


def _oracle(py, puv, y, uv):
    tiles = geo.synthesis_tiles(H, W, LH, LW, (640, 128), geo.image_region_grid(H, W, 2, 3))
    with og.fast_convs():
        return og.synthesize(py, puv, "hop", y, uv, H, W, tiles, 2, 2)


@pytest.fixture(scope="module")
def he05():
    """The He x 0.5 workload and its oracle planes (computed once for the module)."""
    py, puv, y, uv = _workload(5, 0.5)
    return py, puv, y, uv, _oracle(py, puv, y, uv)


def step_stats(got_q, want_q):
    d = np.abs(got_q.astype(np.int32) - want_q.astype(np.int32))
    return int(d.max()), int(np.count_nonzero(d)), d.size


def test_config5_he05_meets_the_8bit_and_10bit_gate(he05):
    eng = nn.Engine(0, "f32")
    py, puv, y, uv, want = he05
    got = _gpu(eng, py, puv, y, uv, 0)
    got10 = _gpu(eng, py, puv, y, uv, 10)
    for name, g, wv, g10 in zip("yuv", got, want, got10):
        err = float(np.max(np.abs(g - wv)))
        s8 = step_stats(oracle.quantize_plane(g, 8), oracle.quantize_plane(wv, 8))
        s10 = step_stats(g10, oracle.quantize_plane(wv, 10))
        print(f"config 5 He x 0.5 {name}: max abs {err:.2e} of 255; 8-bit max step {s8[0]}, "
              f"{s8[1]} of {s8[2]} differ; 10-bit max step {s10[0]}, {s10[1]} of {s10[2]} differ")
        assert err <= 0.05
        for mx, n, size in (s8, s10):
            assert mx <= 1 and n <= 5e-4 * size
    eng.close()


def test_config5_bench_weights_10bit():
    """The benchmarked workload itself: seed 1, He-normal gain 1, 10-bit planes."""
    from test_conditioning import nudge
    eng = nn.Engine(0, "f32")
    py, puv, y, uv = _workload(1, 1.0)
    got = _gpu(eng, py, puv, y, uv, 10)
    want = _oracle(py, puv, y, uv)
    spread = _oracle(nudge(py), nudge(puv, 1), y, uv)
    for name, g, wv, sp in zip("yuv", got, want, spread):
        wq = oracle.quantize_plane(wv, 10)
        mx, n, size = step_stats(g, wq)
        smx, sn, _ = step_stats(oracle.quantize_plane(sp, 10), wq)
        sat = float(np.mean((wv <= 0) | (wv >= 255)))
        print(f"config 5 bench weights {name}: GPU vs oracle 10-bit max step {mx}, {n} of {size} "
              f"differ ({n / size:.2e}); oracle vs oracle(+-1 ulp weights) max step {smx}, {sn} "
              f"differ; oracle saturated fraction {sat:.3f}")
        # The gate's fraction, or 3x the oracle's own spread where that alone exceeds it.
        assert n <= max(5e-4 * size, 3 * sn)
    eng.close()


@pytest.mark.parametrize("prec", ["f16", "bf16"])
def test_config5_16bit_psnr(he05, prec):
    """The 16-bit paths have no gate (the reference's own f16-weight study fails its 1/5000
    gate); their PSNR against the fp32 oracle on the He x 0.5 config-5 picture is printed and
    held above a floor."""
    eng = nn.Engine(0, prec)
    py, puv, y, uv, want = he05
    got = _gpu(eng, py, puv, y, uv, 0)
    for name, g, wv in zip("yuv", got, want):
        mse = float(np.mean((g.astype(np.float64) - wv) ** 2))
        psnr = 99.0 if mse == 0 else 10 * np.log10(255.0 ** 2 / mse)
        mx, n, size = step_stats(oracle.quantize_plane(g, 8), oracle.quantize_plane(wv, 8))
        print(f"config 5 He x 0.5 {prec} {name}: PSNR {psnr:.2f} dB vs the fp32 oracle; 8-bit "
              f"max step {mx}, {n / size:.2%} of samples differ")
        assert np.isfinite(g).all() and psnr >= (35.0 if prec == "f16" else 28.0)
    eng.close()


@pytest.mark.parametrize("prec", ["f32", "bf16"])
def test_config5_output_does_not_depend_on_the_batching(prec):
    """Every kernel choice is either made from one batch item's geometry or sums each output in
    the same order as its alternatives, so a tile's planes must not change with the batch it runs
    in: the 24-tile picture (four batches of 6) against two 12-tile pictures of 3 tiles per shape
    (batches of 3, so other launch grids and tile shapes), compared bit for bit on each tile's
    core (float planes), in f32 and in bf16."""
    py, puv, y, uv = _workload(5, 0.5)
    eng = nn.Engine(0, prec)
    tiles = model.synthesis_tiles(H, W, LH, LW, (640, 128), (2, 3))
    prim = model.SynthesisPrimary.load(py, "hop", eng)
    sec = model.SynthesisSecondary.load(puv, "hop", eng)
    full = model.synthesize(eng, prim, sec, y, uv, H, W, tiles, 2, 2, bit_depth=0, lanes=4)
    by_shape = {}
    for t in tiles:
        by_shape.setdefault((t.image.height, t.image.width), []).append(t)
    assert sorted(len(v) for v in by_shape.values()) == [6, 6, 6, 6]
    for half in (0, 1):
        sub = [t for v in by_shape.values() for t in v[half::2]]
        got = model.synthesize(eng, prim, sec, y, uv, H, W, sub, 2, 2, bit_depth=0, lanes=4)
        for t in sub:
            c = t.core
            assert c.x % 2 == 0 and c.y % 2 == 0 and c.width % 2 == 0 and c.height % 2 == 0
            rects = [(full[0], got[0], c.y, c.x, c.height, c.width)]
            rects += [(f, g, c.y // 2, c.x // 2, c.height // 2, c.width // 2) for f, g in zip(full[1:], got[1:])]
            for f, g, r0, c0, h, w in rects:
                a = f[r0:r0 + h, c0:c0 + w]
                b = g[r0:r0 + h, c0:c0 + w]
                assert a.size > 0 and np.array_equal(a.view(np.uint32), b.view(np.uint32)), (half, c)
    eng.close()
