"""GPU parity of the analysis transforms (src/model/analysis.rs, encoder side) through the
C-ABI against the CPU oracle: fp32 within 1e-4 of the output's range (MFMA convolutions reorder
the sums, as in the synthesis), the index-map closed form bit for bit (which pins the replicate
padding and the strides), feature clipping, nets built from checkpoints, and the refusals."""

import io

import numpy as np
import pytest
import torch

import oracle.graphs as og
from tests.test_analysis_oracle import index_map_closed_form, index_map_params
from zenjpegai_amd import _lib, model, nn, synth
from zenjpegai_amd.weights import Checkpoint

pytestmark = pytest.mark.gpu

TOL = 1e-4


@pytest.fixture(scope="module")
def engines():
    return {p: nn.Engine(0, p) for p in ("f32", "f16", "bf16")}


def _close(got, want, tol=TOL):
    err = float(np.max(np.abs(got - want)))
    ref = float(np.max(np.abs(want)))
    assert err <= tol * ref, (err, ref)
    return err / ref


def _cls(component):
    return model.AnalysisPrimary if component == "y" else model.AnalysisSecondary


def _oracle(component):
    return og.analysis_primary if component == "y" else og.analysis_secondary


@pytest.mark.parametrize("op", ["bop", "hop"])
@pytest.mark.parametrize("component,h,w", [("y", 64, 64), ("y", 70, 90), ("uv", 32, 48), ("uv", 35, 21)])
def test_analysis_matches_oracle(engines, op, component, h, w):
    eng = engines["f32"]
    p = synth.random_analysis_params(op, component, seed=41, gain=0.5)
    x = synth.picture(41, f"{op}{component}", 1 if component == "y" else 12, h, w)
    got = _cls(component).load(p, op, eng).forward(eng, x)
    want = _oracle(component)(p, op, x)
    assert got.shape == want.shape
    r = _close(got, want)
    print(f"analysis {op} {component} {h}x{w}: max rel {r:.2e}")


@pytest.mark.parametrize("component,h,w", [("y", 70, 90), ("y", 33, 47), ("uv", 21, 35)])
def test_index_map_analysis_is_bit_exact(engines, component, h, w):
    eng = engines["f32"]
    p = index_map_params("bop", component)
    c = 1 if component == "y" else 12
    x = synth.picture(8, f"im{component}", c, h, w)
    got = _cls(component).load(p, "bop", eng).forward(eng, x)
    want = index_map_closed_form(x, 4 if component == "y" else 3)
    assert np.array_equal(got[:c], want)
    assert not np.any(got[c:])


@pytest.mark.parametrize("op", ["bop", "hop"])
def test_clip_thres_lists(engines, op):
    eng = engines["f32"]
    p = synth.random_analysis_params(op, "y", seed=42, gain=0.5)
    x = synth.picture(42, "clip", 1, 48, 64)
    s = "H" if op == "hop" else "B"
    for k, n in ((1, 100), (3, 128), (4, 160), (5, 90)):
        p[f"clip_thres.E{k}{s}.MinList"] = np.full(n, -0.05, np.float32)
        p[f"clip_thres.E{k}{s}.MaxList"] = np.full(n + 3, 0.05, np.float32)
    net = model.AnalysisPrimary.load(p, op, eng)
    _close(net.forward(eng, x), og.analysis_primary(p, op, x))
    clipped = net.forward(eng, x, clip=True)
    _close(clipped, og.analysis_primary(p, op, x, clip=True))
    assert np.all(np.abs(clipped[:90]) <= 0.05)


def test_analysis_from_a_checkpoint_is_the_dict_net(engines):
    eng = engines["f32"]
    p = synth.random_analysis_params("hop", "uv", seed=43, gain=0.5)
    b = io.BytesIO()
    sd = {k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in p.items()}
    sd["clip_thres"] = {"E5H": {"MinList": [-0.02] * 96, "MaxList": [0.02] * 96}}
    torch.save(sd, b)
    ck = Checkpoint.parse(b.getvalue())
    x = synth.picture(43, "ck", 12, 32, 40)
    a = model.AnalysisSecondary.load(ck, "hop", eng)
    q = dict(p, **{"clip_thres.E5H.MinList": np.full(96, -0.02, np.float32),
                   "clip_thres.E5H.MaxList": np.full(96, 0.02, np.float32)})
    d = model.AnalysisSecondary.load(q, "hop", eng)
    for clip in (False, True):
        assert np.array_equal(a.forward(eng, x, clip), d.forward(eng, x, clip))


@pytest.mark.parametrize("prec", ["bf16", "f16"])
def test_analysis_16bit_storage(engines, prec):
    """16-bit activations and weights, f32 accumulation: no gate, as for the synthesis; the
    relative error against the fp32 oracle is printed and bounded loosely."""
    eng = engines[prec]
    p = synth.random_analysis_params("hop", "y", seed=44, gain=0.5)
    x = synth.picture(44, "16", 1, 64, 96)
    got = model.AnalysisPrimary.load(p, "hop", eng).forward(eng, x)
    want = og.analysis_primary(p, "hop", x)
    rel = float(np.max(np.abs(got - want)) / np.max(np.abs(want)))
    print(f"analysis hop y {prec}: max rel {rel:.2e}")
    assert rel < (5e-2 if prec == "bf16" else 1e-2)


def test_refusals(engines):
    eng = engines["f32"]
    p = synth.random_analysis_params("bop", "y", seed=45)
    with pytest.raises(_lib.HipError) as e:
        model.AnalysisPrimary.load(p, "sop", eng)
    assert e.value.code == _lib.E_INVALID_ARGUMENT and "SOP" in str(e.value)
    net = model.AnalysisPrimary.load(p, "bop", eng)
    with pytest.raises(_lib.HipError):
        net.forward(eng, synth.picture(1, "bad", 12, 32, 32))  # luma takes one plane
    q = dict(p)
    q.pop("act2.conv2.weight")
    with pytest.raises(_lib.HipError) as e:
        model.AnalysisPrimary.load(q, "bop", eng)
    assert e.value.code == _lib.E_MODEL
