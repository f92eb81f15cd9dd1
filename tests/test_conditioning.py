"""Conditioning of the BASELINE workloads, shown with the oracle alone (CPU): the reference's own
f32 computation, rerun with every weight moved by one ulp (``nextafter`` towards a random
side), against itself. One ulp per weight perturbs each sum by about as much as reordering its
terms does, so this is the spread any correct f32 implementation with another summation order
(the MFMA kernels) must expect.

* He-normal gain 1 (the BASELINE spec, config 4 and the bench's config-5 weights): activations
  grow to ~1e4-1e5 before ``denormalize`` (x * 128 + 127.5, clamped), nearly every sample
  saturates, and the few samples whose pre-denormalize value ends up near the clamp edges --
  small differences of large terms -- flip by many steps, also between the oracle and itself.
  The north-star "one step in 0.05 %" gate is therefore not attainable there by any other
  summation order; the GPU tests hold the gain-1 workloads to the 0.05 % fraction bound and to
  the oracle's own spread under this perturbation.
* He-normal x 0.5: the outputs span the range, and the perturbed oracle meets the gate.
Reference gate: tests/decode_ref.rs:157-190; denormalize: src/model/synthesis.rs:187-192."""

import numpy as np
import pytest

import oracle
import oracle.graphs as og
from oracle import geometry as geo
from zenjpegai_amd import synth


def nudge(params, seed=0):
    """Every conv / transposed-conv weight moved by one ulp towards a random side."""
    rng = np.random.default_rng(seed)
    out = {}
    for k, v in params.items():
        if k.endswith(".weight") and v.ndim == 4:
            side = np.where(rng.random(v.shape) < 0.5, -np.inf, np.inf).astype(np.float32)
            out[k] = np.nextafter(v, side).astype(np.float32)
        else:
            out[k] = v
    return out


def steps(a, b, bits):
    d = np.abs(oracle.quantize_plane(a, bits).astype(np.int32) - oracle.quantize_plane(b, bits).astype(np.int32))
    return int(d.max()), float(np.count_nonzero(d)) / d.size


def config4(gain):
    p = synth.random_params("sop", "y", seed=4, gain=gain)
    y = synth.latent(4, "cfg4/y", 160, 64, 64)
    with og.fast_convs():
        pre = og.primary(p, "sop", y, 1024, 1024, denorm=False)[0]
        pre_n = og.primary(nudge(p), "sop", y, 1024, 1024, denorm=False)[0]
    return pre, pre_n


def config5_tile(gain):
    """The first 704 x 704 tile of config 5 (HOP luma), the bench's seed for gain 1."""
    lh, lw = 135, 240
    tiles = geo.synthesis_tiles(2160, 3840, lh, lw, (640, 128), geo.image_region_grid(2160, 3840, 2, 3))
    t = next(t for t in tiles if (t.image.width, t.image.height) == (704, 704))
    seed = 1 if gain == 1.0 else 5
    p = synth.random_params("hop", "y", seed=seed, gain=gain)
    y = synth.latent(seed, "cfg5/y", 160, lh, lw)
    y = np.ascontiguousarray(y[:, t.latent.y:t.latent.y + t.latent.height, t.latent.x:t.latent.x + t.latent.width])
    with og.fast_convs():
        pre = og.primary(p, "hop", y, t.image.height, t.image.width, denorm=False)[0]
        pre_n = og.primary(nudge(p), "hop", y, t.image.height, t.image.width, denorm=False)[0]
    return pre, pre_n


@pytest.mark.parametrize("case,bits", [("config4", 8), ("config5_tile", 10)])
def test_he_gain1_is_ill_conditioned_in_the_oracle_itself(case, bits):
    pre, pre_n = (config4 if case == "config4" else config5_tile)(1.0)
    a, b = oracle.denormalize(pre), oracle.denormalize(pre_n)
    mx, frac = steps(a, b, bits)
    sat = float(np.mean((a <= 0) | (a >= 255)))
    scale = float(np.max(np.abs(pre)))
    flipped = np.abs(oracle.quantize_plane(a, bits).astype(np.int32) -
                     oracle.quantize_plane(b, bits).astype(np.int32)) > 1
    print(f"{case} He gain 1: oracle vs oracle(weights +-1 ulp): {bits}-bit max step {mx}, "
          f"{frac:.2e} of samples differ; saturated {sat:.3f}; max|pre| {scale:.3g}; "
          f"largest |pre| of a flipped sample {float(np.max(np.abs(pre[flipped]))):.3g}")
    assert sat > 0.9
    assert mx > 1  # the gate's one-step bound fails for the reference computation itself
    assert frac <= 5e-4
    # The flips are differences of large terms: small next to the activations' scale.
    assert float(np.max(np.abs(pre[flipped]))) <= 1e-3 * scale


def test_he_half_gain_meets_the_gate_in_the_oracle_itself():
    pre, pre_n = config4(0.5)
    mx, frac = steps(oracle.denormalize(pre), oracle.denormalize(pre_n), 8)
    print(f"config4 He x 0.5: oracle vs oracle(weights +-1 ulp): max step {mx}, {frac:.2e} differ")
    assert mx <= 1 and frac <= 5e-4
