"""GPU: nets built from parsed checkpoints (zjai_net_create_from_checkpoint,
zjai_latent_model_create_from_checkpoint) are the nets built from the same named arrays -- the
outputs agree bit for bit -- for `.pth` files written by torch.save, packed ZJM1 files inside a
ZJB1 bundle, and ZJB2 (f16-weight) members, whose nets equal nets given the f16-rounded weights
(the upcast is exact; src/weights/packed.rs:36-42)."""

import io

import numpy as np
import pytest
import torch

from zenjpegai_amd import model, nn, synth
from zenjpegai_amd.weights import Checkpoint, PackedBundle, write_bundle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def eng():
    return nn.Engine(0, "f32")


def _pth(params) -> bytes:
    b = io.BytesIO()
    torch.save({k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in params.items()}, b)
    return b.getvalue()


def _containers(params):
    """(label, Checkpoint, the arrays it should be equivalent to)."""
    pth = Checkpoint.parse(_pth(params))
    names = pth.tensor_names()
    bundle = PackedBundle.parse(write_bundle([("m/a.pth", pth.write_zjm(names)),
                                              ("m/b.pth", pth.write_zjm(names, f16=True))], "n"))
    rounded = {k: v.astype(np.float16).astype(np.float32) for k, v in params.items()}
    return [("pth", pth, params), ("zjm1", bundle.checkpoint("m/a.pth"), params),
            ("zjb2-f16", bundle.checkpoint("m/b.pth"), rounded)]


@pytest.mark.parametrize("op", ["sop", "hop"])
def test_primary_from_checkpoint_is_the_dict_net(eng, op):
    p = synth.random_params(op, "y", seed=31, gain=0.5)
    y = nn.BTensor.from_planar(eng, synth.latent(31, f"{op}/y", 160, 4, 6))
    for label, ck, arrays in _containers(p):
        got = model.SynthesisPrimary.load(ck, op, eng).forward(eng, y, 64, 96)
        want = model.SynthesisPrimary.load(arrays, op, eng).forward(eng, y, 64, 96)
        print(f"{op} Y {label}: identical {np.array_equal(got, want)}")
        assert np.array_equal(got, want), label


def test_secondary_from_checkpoint_is_the_dict_net(eng):
    p = synth.random_params("bop", "uv", seed=32, gain=0.5)
    y = nn.BTensor.from_planar(eng, synth.latent(32, "bop/y", 160, 4, 3))
    uv = nn.BTensor.from_planar(eng, synth.latent(32, "bop/uv", 96, 4, 3))
    for label, ck, arrays in _containers(p):
        got = model.SynthesisSecondary.load(ck, "bop", eng).forward(eng, y, uv, 64, 48)
        want = model.SynthesisSecondary.load(arrays, "bop", eng).forward(eng, y, uv, 64, 48)
        assert np.array_equal(got, want), label


@pytest.mark.parametrize("ccs", [0, 1])
def test_latent_model_from_checkpoint_is_the_dict_model(eng, ccs):
    p = synth.random_latent_params(ccs, seed=33, gain=1.0)
    c = synth.LATENT_CHANNELS[ccs]
    z = synth.hyper_latent(33, f"ck{ccs}", c, 4, 6)
    res = synth.residual(33, f"ckr{ccs}", c, 16, 24)
    for label, ck, arrays in _containers(p):
        a = model.LatentModel.load(ck, ccs, eng)
        b = model.LatentModel.load(arrays, ccs, eng)
        assert a.has_context == b.has_context and a.channels == b.channels == c
        psi_a, psi_b = a.hyper_decoder(z, 8, 12), b.hyper_decoder(z, 8, 12)
        assert np.array_equal(psi_a, psi_b), label
        assert np.array_equal(a.decompress(res, psi_a), b.decompress(res, psi_b)), label


def test_a_checkpoint_missing_a_weight_is_a_model_error(eng):
    p = synth.random_params("sop", "y", seed=34)
    p.pop(next(iter(p)))
    with pytest.raises(model.HipError) as e:
        model.SynthesisPrimary.load(Checkpoint.parse(_pth(p)), "sop", eng)
    assert e.value.kind == "Model"
