"""GPU: the allocation-free entry point ``zjai_channel_attention_noalloc`` against
``zjai_channel_attention`` (src/nn/fast/math.rs:512-603), through the C-ABI, bit for bit: two
calls in a row with the second on a smaller map (the shared scratch then holds the first call's
larger contents), in f32, f16 and bf16, dims 128 and 64 and a dim of 8 whose folded weight has
padded rows and columns. A map beyond the scratch returns LimitExceeded before any launch.

The caller-owned device buffers come from the HIP runtime the library itself links
(libamdhip64.so.7, via ctypes)."""

import ctypes

import numpy as np
import pytest

from zenjpegai_amd import _lib, nn, synth

pytestmark = pytest.mark.gpu

H2D, D2H = 1, 2


def _hip():
    _lib.lib()  # loads libzjai_hip.so and with it the HIP runtime it links
    h = ctypes.CDLL("libamdhip64.so.7")
    h.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
    h.hipFree.argtypes = [ctypes.c_void_p]
    h.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    for f in (h.hipMalloc, h.hipFree, h.hipMemcpy, h.hipDeviceSynchronize):
        f.restype = ctypes.c_int
    return h


class DevBuf:
    def __init__(self, hip, nbytes):
        self.hip, self.n = hip, nbytes
        self.p = ctypes.c_void_p()
        assert hip.hipMalloc(ctypes.byref(self.p), nbytes) == 0

    def put(self, arr):
        a = np.ascontiguousarray(arr)
        assert a.nbytes == self.n
        assert self.hip.hipMemcpy(self.p, a.ctypes.data, self.n, H2D) == 0

    def get(self, dtype, shape):
        a = np.empty(shape, dtype)
        assert a.nbytes == self.n
        assert self.hip.hipMemcpy(a.ctypes.data, self.p, self.n, D2H) == 0
        return a

    def free(self):
        self.hip.hipFree(self.p)


def _storage_exact(x, prec):
    """Values exactly representable in the storage type, and their raw storage array."""
    if prec == "f32":
        return x, x
    if prec == "f16":
        v = x.astype(np.float16)
        return v.astype(np.float32), v
    bits = x.view(np.uint32) & np.uint32(0xFFFF0000)
    return bits.view(np.float32), (bits >> np.uint32(16)).astype(np.uint16)


def _to_f32(raw, prec):
    if prec == "f32":
        return raw
    if prec == "f16":
        return raw.astype(np.float32)
    return (raw.astype(np.uint32) << np.uint32(16)).view(np.float32)


def _run_both(eng, hip, dim, heads, h, w, prec, seed):
    c3 = 3 * dim
    x = synth.normal(seed, f"noalloc/{dim}/{h}x{w}", (c3, h, w), 1.0)
    x, raw = _storage_exact(x, prec)
    temp = np.linspace(0.5, 2.0, heads).astype(np.float32)
    want = nn.channel_attention(eng, nn.BTensor.from_planar(eng, x), heads, temp).to_planar()
    es = 4 if prec == "f32" else 2
    d_q, d_t, d_o = DevBuf(hip, c3 * h * w * es), DevBuf(hip, heads * 4), DevBuf(hip, dim * h * w * es)
    try:
        d_q.put(np.ascontiguousarray(raw.transpose(1, 2, 0)))
        d_t.put(temp)
        assert hip.hipDeviceSynchronize() == 0
        rc = _lib.lib().zjai_channel_attention_noalloc(eng.handle, d_q.p, c3, h, w, heads, d_t.p,
                                                       _lib.PRECISIONS[prec], d_o.p)
        assert rc == _lib.OK, rc
        eng.sync()
        assert hip.hipDeviceSynchronize() == 0
        got = _to_f32(d_o.get(raw.dtype, (h, w, dim)), prec).transpose(2, 0, 1)
    finally:
        for b in (d_q, d_t, d_o):
            b.free()
    return got, want


@pytest.mark.parametrize("prec", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("dim,heads", [(128, 4), (64, 4), (8, 2)])
def test_noalloc_attention_equals_the_allocating_entry_point(prec, dim, heads):
    eng = nn.Engine(0, prec)
    hip = _hip()
    for h, w, seed in ((96, 80, 1), (20, 12, 2)):  # the second call is smaller
        got, want = _run_both(eng, hip, dim, heads, h, w, prec, seed)
        assert got.shape == want.shape
        assert np.isfinite(want).all()
        assert np.array_equal(got, want), (prec, dim, h, w, float(np.max(np.abs(got - want))))
    eng.close()


def test_noalloc_attention_rejects_a_map_beyond_the_scratch():
    """Checked on the host before any launch: 1024 x 1024 positions at dim 128 need ~71 MB of
    Gram partials, more than the 16 MiB scratch; dim 640 exceeds the Gram kernel's LDS stage.
    The buffers are never touched."""
    eng = nn.Engine(0, "f32")
    hip = _hip()
    d = DevBuf(hip, 4096)
    try:
        rc = _lib.lib().zjai_channel_attention_noalloc(eng.handle, d.p, 384, 1024, 1024, 4, d.p,
                                                       _lib.F32, d.p)
        assert rc == _lib.E_LIMIT
        rc = _lib.lib().zjai_channel_attention_noalloc(eng.handle, d.p, 384, 16, 16, 5, d.p,
                                                       _lib.F32, d.p)
        assert rc == _lib.E_INVALID_ARGUMENT
        # dim 640 (20 heads of 32): the Gram kernel's LDS stage would exceed 160 KB; refused as
        # Unsupported before the padding fill or any other launch.
        rc = _lib.lib().zjai_channel_attention_noalloc(eng.handle, d.p, 1920, 4, 4, 20, d.p,
                                                       _lib.F32, d.p)
        assert rc == _lib.E_UNSUPPORTED
    finally:
        d.free()
    eng.close()
