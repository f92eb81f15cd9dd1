"""GPU parity of the latent reconstruction (src/decoder/reconstruct.rs:81-234): the hyper-decoder
(src/model/hyper_decoder.rs), the multi-stage context model (src/model/mcm.rs) and the region
driver, through the C-ABI, against the CPU oracle.

fp32 path: every network is a chain of MFMA convolutions, so the bar is the per-layer one of
the synthesis (max |gpu - oracle| <= 1e-4 x max |oracle|), applied to the networks' outputs
(psi, and the predicted means y_hat - residual). Pure data movement (the up-shuffled psi plus
residual) and the index-map nets of the oracle's closed-form pins are bit-exact."""

import numpy as np
import pytest

import oracle.graphs as og
from oracle import geometry as geo
from tests.test_latent_oracle import _delta_params, _psi_closed_form, _y_closed_form
from zenjpegai_amd import _lib, model, nn, synth

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _ceil(a, b):
    return -(-a // b)


@pytest.fixture(scope="module")
def eng():
    e = nn.Engine(0, "f32")
    yield e
    e.close()


def _close(got, want, tol=TOL):
    err = float(np.max(np.abs(got - want))) if want.size else 0.0
    ref = float(np.max(np.abs(want))) if want.size else 0.0
    assert err <= tol * max(ref, 1e-30), (err, ref)
    return err / max(ref, 1e-30)


def _sizes(ccs, height, width):
    if ccs == 0:
        return _ceil(height, 16), _ceil(width, 16), _ceil(height, 64), _ceil(width, 64)
    h2, w2 = 2 * _ceil(height, 2), 2 * _ceil(width, 2)
    return _ceil(_ceil(height, 2), 8), _ceil(_ceil(width, 2), 8), _ceil(h2, 64), _ceil(w2, 64)


def _mr(r):
    if r is None:
        return None
    return model.Regions(r.num_ver, r.num_hor, r.independent, r.hyper_decoder_overlap, r.mcm_overlap)


@pytest.mark.parametrize("ccs", [0, 1])
@pytest.mark.parametrize("zh,zw,oh,ow", [(4, 6, 8, 12), (5, 7, 9, 13), (3, 3, 6, 5)])
def test_hyper_decoder_matches_oracle(eng, ccs, zh, zw, oh, ow):
    p = synth.random_latent_params(ccs, seed=21, gain=1.0)
    c = synth.LATENT_CHANNELS[ccs]
    m = model.LatentModel.load(p, ccs, eng)
    assert (m.channels, m.has_context) == (c, True)
    z = synth.hyper_latent(21, f"hz{ccs}", c, zh, zw)
    got = m.hyper_decoder(z, oh, ow)
    want = og.hyper_decoder(p, z, oh, ow)
    assert got.shape == want.shape == (4 * c, oh, ow)
    rel = _close(got, want)
    print(f"hyper-decoder ccs {ccs} {zh}x{zw} -> {oh}x{ow}: max rel err {rel:.2e}")


@pytest.mark.parametrize("ccs", [0, 1])
@pytest.mark.parametrize("h,w", [(16, 24), (15, 23), (9, 2)])
def test_context_model_matches_oracle(eng, ccs, h, w):
    p = synth.random_latent_params(ccs, seed=22, gain=1.0)
    c = synth.LATENT_CHANNELS[ccs]
    m = model.LatentModel.load(p, ccs, eng)
    res = synth.residual(22, f"cr{ccs}", c, h, w)
    psi = synth.laplace(22, f"cpsi{ccs}", (4 * c, _ceil(h, 2), _ceil(w, 2)), 1.0)
    got = m.decompress(res, psi)
    want = og.context_decompress(p, res, psi)
    rel = _close(got - res, want - res)
    print(f"context model ccs {ccs} {h}x{w}: max rel err of the means {rel:.2e}")


def test_no_context_model_is_upshuffle_plus_residual_exactly(eng):
    p = synth.random_latent_params(0, seed=23, context=False)
    m = model.LatentModel.load(p, 0, eng)
    assert not m.has_context
    res = synth.residual(23, "ur", 160, 15, 23)
    psi = synth.laplace(23, "upsi", (640, 8, 12), 2.0)
    got = m.decompress(res, psi)
    assert np.array_equal(got, og.upshuffle_psi(psi, 15, 23) + res)


@pytest.mark.parametrize("ccs", [0, 1])
@pytest.mark.parametrize("height,width,regions", [
    (256, 384, None),
    (1000, 1400, None),
    (1024, 1536, geo.Regions(2, 3, True)),
    (1024, 1536, geo.Regions(2, 2, False, 1, 4)),
    (900, 1300, geo.Regions(2, 2, False, 2, 1)),
])
def test_reconstruct_latent_matches_oracle(eng, ccs, height, width, regions):
    p = synth.random_latent_params(ccs, seed=24, gain=1.0)
    c = synth.LATENT_CHANNELS[ccs]
    lh, lw, zh, zw = _sizes(ccs, height, width)
    m = model.LatentModel.load(p, ccs, eng)
    z = synth.hyper_latent(24, f"rz{ccs}", c, zh, zw)
    res = synth.residual(24, f"rr{ccs}", c, lh, lw)
    psi, y = m.reconstruct(height, width, _mr(regions), z, res)
    want_psi, want_y = og.reconstruct_latent(p, ccs, height, width, regions, z, res)
    r1 = _close(psi, want_psi)
    r2 = _close(y - res, want_y - res)
    print(f"reconstruct ccs {ccs} {height}x{width} {regions}: psi {r1:.2e}, means {r2:.2e}")


@pytest.mark.parametrize("ccs", [0, 1])
@pytest.mark.parametrize("height,width,regions", [
    (1024, 1536, None),
    (1024, 1536, geo.Regions(2, 3, True)),
    (1024, 1536, geo.Regions(2, 2, False, 1, 4)),
    # nine regions of four shapes: corner, edge and interior regions share batches
    (1536, 1536, geo.Regions(3, 3, False, 1, 4)),
    (2048, 2048, geo.Regions(4, 4, True)),
])
def test_reconstruct_latent_with_index_map_weights_is_exact(eng, ccs, height, width, regions):
    """The oracle's closed-form pins run on the GPU: identity weights make every MFMA sum a
    single product plus exact zeros, so psi and y_hat are bit-exact."""
    lh, lw, zh, zw = _sizes(ccs, height, width)
    c = synth.LATENT_CHANNELS[ccs]
    p = _delta_params(c)
    m = model.LatentModel.load(p, ccs, eng)
    z = synth.hyper_latent(25, f"dz{ccs}", c, zh, zw, b=3.0)
    res = synth.residual(25, f"dr{ccs}", c, lh, lw, b=2.0)
    psi, y = m.reconstruct(height, width, _mr(regions), z, res)
    want_psi = _psi_closed_form(z.astype(np.float32), _ceil(lh, 2), _ceil(lw, 2))
    assert np.array_equal(psi, want_psi)
    assert np.array_equal(y, _y_closed_form(want_psi, res))


@pytest.mark.parametrize("prec", ["bf16", "f16"])
def test_reconstruct_latent_16bit_storage(prec):
    """16-bit storage of the networks' activations and weights: no gate (as for the synthesis),
    the means stay within a few percent of the fp32 oracle."""
    e = nn.Engine(0, prec)
    try:
        p = synth.random_latent_params(0, seed=26, gain=1.0)
        lh, lw, zh, zw = _sizes(0, 512, 768)
        m = model.LatentModel.load(p, 0, e)
        z = synth.hyper_latent(26, "bz", 160, zh, zw)
        res = synth.residual(26, "br", 160, lh, lw)
        psi, y = m.reconstruct(512, 768, None, z, res)
        want_psi, want_y = og.reconstruct_latent(p, 0, 512, 768, None, z, res)
        rel_psi = float(np.max(np.abs(psi - want_psi)) / np.max(np.abs(want_psi)))
        rel_y = float(np.max(np.abs((y - res) - (want_y - res))) / np.max(np.abs(want_y - res)))
        print(f"{prec}: psi max rel err {rel_psi:.2e}, means {rel_y:.2e}")
        assert rel_psi < 5e-2 and rel_y < 5e-2
    finally:
        e.close()


def test_latent_errors_are_invalid_arguments(eng):
    p = synth.random_latent_params(1, seed=27)
    m = model.LatentModel.load(p, 1, eng)
    res = synth.residual(27, "er", 96, 8, 8)
    with pytest.raises(_lib.HipError) as e:
        m.decompress(res, np.zeros((384, 5, 4), np.float32))  # psi not ceil(h/2) x ceil(w/2)
    assert e.value.kind == "InvalidArgument"
    with pytest.raises(_lib.HipError) as e:
        m.hyper_decoder(np.zeros((96, 2, 2), np.int8), 5, 4)  # crop larger than 2x
    assert e.value.kind == "InvalidArgument"
    with pytest.raises(_lib.HipError) as e:
        m.reconstruct(128, 128, None, np.zeros((96, 1, 1), np.int8),
                      np.zeros((96, 4, 4), np.float32))  # residual smaller than the latent
    assert e.value.kind == "InvalidArgument"
    bad = dict(p)
    bad["hyper_decoder.conv4.weight"] = bad["hyper_decoder.conv4.weight"][:100]
    with pytest.raises(_lib.HipError) as e:
        model.LatentModel.load(bad, 1, eng)
    assert e.value.kind == "Model"
