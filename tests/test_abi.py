"""CPU tests of the C-ABI library: it loads, exports exactly what include/zjai_hip.h declares,
reports device errors without a GPU, and its host-side tiling geometry equals the oracle's."""

import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from oracle import geometry as geo
from zenjpegai_amd import _lib, model, synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "zjai_hip.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"ZJAI_API\s+int32_t\s+(zjai_\w+)\s*\(", text)))


def _exported():
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    return sorted({l.split()[-1] for l in out.splitlines() if " T " in l})


def test_library_exports_exactly_the_declared_abi():
    declared = _declared()
    assert len(declared) >= 40
    assert _exported() == declared
    assert sorted(_lib.PROTOTYPES) == declared
    L = _lib.lib()
    for name in declared:
        assert getattr(L, name) is not None


def _has_gpu():
    return os.path.exists("/dev/kfd")


@pytest.mark.skipif(_has_gpu(), reason="checks the no-device error path")
def test_context_creation_without_a_gpu_reports_a_device_error():
    L = _lib.lib()
    h = ctypes.c_void_p()
    rc = L.zjai_ctx_create(0, 0, ctypes.byref(h))
    assert rc == _lib.E_DEVICE
    assert not h.value
    msg = _lib.last_error(None)
    assert "device" in msg.lower()
    with pytest.raises(_lib.HipError) as e:
        from zenjpegai_amd import nn
        nn.Engine(0)
    assert e.value.kind == "Device"


def test_null_arguments_are_rejected():
    L = _lib.lib()
    assert L.zjai_ctx_create(0, 0, None) == _lib.E_INVALID_ARGUMENT
    assert L.zjai_sync(None) == _lib.E_INVALID_ARGUMENT
    assert L.zjai_picture_run(None, None) == _lib.E_INVALID_ARGUMENT
    assert L.zjai_ctx_destroy(None) == _lib.OK


def test_context_flags_match_the_header_and_unknown_flags_are_rejected():
    text = open(HEADER).read()
    m = re.search(r"#define\s+ZJAI_CTX_UNFUSED_BLOCKS\s+(0x[0-9a-fA-F]+)u", text)
    assert m and int(m.group(1), 16) == _lib.CTX_UNFUSED_BLOCKS
    m = re.search(r"#define\s+ZJAI_CTX_PHASE_SPLIT_CONVT\s+(0x[0-9a-fA-F]+)u", text)
    assert m and int(m.group(1), 16) == _lib.CTX_PHASE_SPLIT_CONVT
    L = _lib.lib()
    h = ctypes.c_void_p()
    assert L.zjai_ctx_create(0, 0x80, ctypes.byref(h)) == _lib.E_INVALID_ARGUMENT
    assert not h.value
    assert "flags" in _lib.last_error(None)


def _as_oracle(t):
    A = geo.Area
    return geo.SynthesisTile(A(t.image.x, t.image.y, t.image.width, t.image.height),
                             A(t.latent.x, t.latent.y, t.latent.width, t.latent.height),
                             A(t.core.x, t.core.y, t.core.width, t.core.height), t.core_offset)


@pytest.mark.parametrize("h,w,tiling", [
    (888, 560, None), (1400, 2096, (1024, 64)), (1024, 1024, (640, 64)),
    (2048, 2048, (1024, 64)), (720, 1280, (512, 128)), (300, 500, (256, 64)),
])
def test_tiles_equal_the_oracle(h, w, tiling):
    lh, lw = -(-h // 16), -(-w // 16)
    got = [_as_oracle(t) for t in model.synthesis_tiles(h, w, lh, lw, tiling)]
    assert got == geo.synthesis_tiles(h, w, lh, lw, tiling)


@pytest.mark.parametrize("h,w,rows,cols", [(2160, 3840, 2, 3), (1400, 2096, 1, 2),
                                           (1024, 2048, 1, 2), (3000, 3000, 3, 3)])
def test_region_tiles_equal_the_oracle(h, w, rows, cols):
    lh, lw = -(-h // 16), -(-w // 16)
    tiling = geo.synthesis_tiling(h, w, (rows, cols)) or (min(h, w), 128)
    regions = geo.image_region_grid(h, w, rows, cols)
    want = geo.synthesis_tiles(h, w, lh, lw, tiling, regions)
    got = [_as_oracle(t) for t in model.synthesis_tiles(h, w, lh, lw, tiling, (rows, cols))]
    assert got == want
    assert sum(t.core.width * t.core.height for t in got) == h * w


def test_region_tiles_match_reference_kat():
    """src/tools/tiles.rs:522-556 through the library (two regions split at x = 1024)."""
    t = model.synthesis_tiles(1400, 2096, 88, 131, (640, 128), (1, 2))
    assert (t[6].latent.x, t[6].latent.y, t[6].latent.width, t[6].latent.height) == (76, 36, 48, 48)
    assert (t[6].core.x, t[6].core.y, t[6].core.width, t[6].core.height) == (1280, 640, 640, 640)
    assert t[6].core_offset == (64, 64)
    assert len(t) == 12


def test_degenerate_tiling_is_an_invalid_argument():
    with pytest.raises(_lib.HipError) as e:
        model.synthesis_tiles(1400, 2096, 88, 131, (64, 64))
    assert e.value.kind == "InvalidArgument"
    assert "overlap" in str(e.value)


def test_synthetic_generator_is_deterministic_and_shaped():
    a = synth.random_params("hop", "y", seed=5)
    b = synth.random_params("hop", "y", seed=5)
    assert a.keys() == b.keys()
    for k in a:
        assert np.array_equal(a[k], b[k])
    w = a["CAB.residual_trunk.0.conv1.weight"]
    assert w.shape == (128, 128, 3, 3)
    assert abs(float(w.std()) - np.sqrt(2 / 1152)) < 0.002
    lat = synth.latent(1, "y", 160, 8, 8)
    assert np.array_equal(lat, np.round(lat)) and lat.dtype == np.float32
    u = synth.uniform(1, "u", (100000,), -1, 1)
    assert -1 <= u.min() and u.max() < 1 and abs(u.mean()) < 0.01
