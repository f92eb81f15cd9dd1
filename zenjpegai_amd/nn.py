"""Operator-level surface of the HIP backend, mirroring the reference's ``nn`` API
(``src/nn/mod.rs``, ``src/nn/fast/{mod,layers,math,tensor}.rs``): ``Conv2d`` /
``ConvTranspose2d`` parameter objects, an ``Engine``, device ``BTensor`` activations,
``ConvLayer`` / ``ConvTransposeLayer`` with ``forward(eng, x)``, and the in-place elementwise
operations. Every call goes through the C-ABI of ``libzjai_hip.so``.
"""

from __future__ import annotations

import ctypes
import weakref
from dataclasses import dataclass, field

import numpy as np

from . import _lib
from ._lib import HipError, check, lib

_f32p = ctypes.POINTER(ctypes.c_float)


def _fp(a: np.ndarray | None):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_f32p)


def _f32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


@dataclass
class Conv2d:
    """``nn::Conv2d`` (src/nn/mod.rs:56-132): weight ``[out][in/groups][kh][kw]``."""
    in_ch: int
    out_ch: int
    kernel: tuple
    stride: int
    pad: tuple
    groups: int
    weight: np.ndarray
    bias: np.ndarray | None = None

    def __post_init__(self):
        kh, kw = self.kernel
        if (self.groups <= 0 or self.in_ch % self.groups or self.out_ch % self.groups
                or self.stride <= 0 or kh <= 0 or kw <= 0):
            raise HipError(_lib.E_MODEL, "conv2d: inconsistent channel/group/kernel configuration")
        self.weight = _f32(self.weight).reshape(self.out_ch, self.in_ch // self.groups, kh, kw)
        self.bias = _f32(self.bias)
        if self.bias is not None and self.bias.shape != (self.out_ch,):
            raise HipError(_lib.E_MODEL, "conv2d: bias size does not match out_ch")

    def out_size(self, h, w):
        kh, kw = self.kernel
        return ((h + 2 * self.pad[0] - kh) // self.stride + 1,
                (w + 2 * self.pad[1] - kw) // self.stride + 1)


@dataclass
class ConvTranspose2d:
    """``nn::ConvTranspose2d`` (src/nn/mod.rs:134-198): weight ``[in][out][k][k]``."""
    in_ch: int
    out_ch: int
    k: int
    stride: int
    pad: int
    out_pad: int
    weight: np.ndarray
    bias: np.ndarray | None = None

    def __post_init__(self):
        if self.stride <= 0 or self.k <= 0 or self.pad >= self.k or self.out_pad >= self.stride:
            raise HipError(_lib.E_MODEL, "conv_transpose2d: unsupported geometry")
        self.weight = _f32(self.weight).reshape(self.in_ch, self.out_ch, self.k, self.k)
        self.bias = _f32(self.bias)

    def out_size(self, h, w):
        f = lambda n: (n - 1) * self.stride + self.k + self.out_pad - 2 * self.pad
        return f(h), f(w)


class Engine:
    """The HIP counterpart of ``nn::fast::Engine`` (src/nn/fast/mod.rs:128-172): one context
    (device + stream) and the precision layers are packed for ("f32", "f16" or "bf16")."""

    def __init__(self, device: int = 0, precision: str = "f32", flags: int = 0):
        """``flags``: 0 or an OR of ``_lib.CTX_*`` (``CTX_UNFUSED_BLOCKS``: the transformer
        blocks as separate kernels instead of the fused ones every precision uses)."""
        self.precision = precision
        self.dtype = _lib.PRECISIONS[precision]
        self._h = ctypes.c_void_p()
        check(lib().zjai_ctx_create(device, flags, ctypes.byref(self._h)), None)

    @property
    def handle(self):
        return self._h

    def sync(self):
        check(lib().zjai_sync(self._h), self._h)

    def host_array(self, shape, dtype=np.float32) -> np.ndarray:
        """A zeroed numpy array in page-locked host memory (``zjai_host_alloc``), for transfer
        buffers reused across pictures; freed with the array (``zjai_host_free``, which needs no
        context, so the array may outlive the engine)."""
        dt = np.dtype(dtype)
        n = int(np.prod(shape)) * dt.itemsize
        p = ctypes.c_void_p()
        check(lib().zjai_host_alloc(self._h, max(n, 1), ctypes.byref(p)), self._h)
        buf = (ctypes.c_byte * max(n, 1)).from_address(p.value)
        arr = np.frombuffer(buf, dtype=np.uint8, count=n).view(dt).reshape(shape)
        arr[...] = 0
        weakref.finalize(buf, lib().zjai_host_free, None, p)
        return arr

    def set_stop(self, stop: bool):
        check(lib().zjai_set_stop(self._h, 1 if stop else 0), self._h)

    def stats(self) -> dict:
        s = _lib.ZjaiStats()
        check(lib().zjai_get_stats(self._h, ctypes.byref(s)), self._h)
        return {k: getattr(s, k) for k, _ in s._fields_}

    def profile_begin(self):
        """Start bracketing every launch with HIP events (see ``zjai_profile_begin``)."""
        check(lib().zjai_profile_begin(self._h), self._h)

    def profile_end(self, cap: int = 1 << 16) -> list:
        """Stop profiling; returns ``[(kernel name, flops, bytes, ms)]`` per launch."""
        recs = (_lib.ZjaiProfRecord * cap)()
        n = ctypes.c_int32()
        check(lib().zjai_profile_end(self._h, recs, cap, ctypes.byref(n)), self._h)
        return [(r.name.decode(), r.flops, r.bytes, r.ms) for r in recs[:min(n.value, cap)]]

    def release_buffers(self):
        check(lib().zjai_release_buffers(self._h), self._h)

    def set_memory_limit(self, nbytes: int):
        """Admission bound (``Limits::max_memory_bytes``): pictures whose nets plus
        ``model.estimate_picture_memory`` exceed ``nbytes`` are refused with ``E_LIMIT`` before
        anything is allocated; 0 disables the check (``zjai_ctx_set_memory_limit``)."""
        check(lib().zjai_ctx_set_memory_limit(self._h, nbytes), self._h)

    def inject_failure(self, what: int, after: int = 0):
        """Fail the next allocation (``_lib.FAIL_ALLOC``) or launch (``_lib.FAIL_LAUNCH``)
        after ``after`` successful ones, from the host (``zjai_inject_failure``)."""
        check(lib().zjai_inject_failure(self._h, what, after), self._h)

    def close(self):
        if self._h:
            lib().zjai_ctx_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class BTensor:
    """A device activation (``nn::fast::BTensor``, src/nn/fast/tensor.rs:145-155), NHWC."""

    def __init__(self, eng: Engine, handle: ctypes.c_void_p):
        self.eng = eng
        self._h = handle
        c, h, w, p = (ctypes.c_int32() for _ in range(4))
        check(lib().zjai_tensor_shape(handle, ctypes.byref(c), ctypes.byref(h), ctypes.byref(w),
                                      ctypes.byref(p)), eng.handle)
        self.c, self.h, self.w, self.dtype = c.value, h.value, w.value, p.value

    @classmethod
    def from_planar(cls, eng: Engine, x: np.ndarray) -> "BTensor":
        x = _f32(x)
        c, h, w = x.shape
        out = ctypes.c_void_p()
        check(lib().zjai_tensor_from_planar(eng.handle, _fp(x), c, h, w, eng.dtype,
                                            ctypes.byref(out)), eng.handle)
        return cls(eng, out)

    @classmethod
    def zeros(cls, eng: Engine, c: int, h: int, w: int) -> "BTensor":
        out = ctypes.c_void_p()
        check(lib().zjai_tensor_create(eng.handle, c, h, w, eng.dtype, ctypes.byref(out)),
              eng.handle)
        return cls(eng, out)

    @classmethod
    def cat(cls, parts) -> "BTensor":
        eng = parts[0].eng
        arr = (ctypes.c_void_p * len(parts))(*[p._h for p in parts])
        out = ctypes.c_void_p()
        check(lib().zjai_tensor_cat(eng.handle, arr, len(parts), ctypes.byref(out)), eng.handle)
        return cls(eng, out)

    @property
    def shape(self):
        return (self.c, self.h, self.w)

    def to_planar(self) -> np.ndarray:
        out = np.empty((self.c, self.h, self.w), np.float32)
        check(lib().zjai_tensor_to_planar(self.eng.handle, self._h, _fp(out), out.size),
              self.eng.handle)
        return out

    def crop(self, h: int, w: int) -> "BTensor":
        out = ctypes.c_void_p()
        check(lib().zjai_tensor_crop(self.eng.handle, self._h, h, w, ctypes.byref(out)),
              self.eng.handle)
        return BTensor(self.eng, out)

    def __del__(self):
        try:
            if self._h:
                lib().zjai_tensor_destroy(self._h)
                self._h = None
        except Exception:
            pass


class _Layer:
    def __init__(self, eng: Engine, handle):
        self.eng = eng
        self._h = handle

    def forward(self, eng: Engine, x: BTensor) -> BTensor:
        out = ctypes.c_void_p()
        check(lib().zjai_conv_forward(eng.handle, self._h, x._h, ctypes.byref(out)), eng.handle)
        return BTensor(eng, out)

    def forward_fused(self, eng: Engine, x: BTensor, act=_lib.ACT_NONE, res=_lib.RES_NONE,
                      r1: BTensor | None = None, r2: BTensor | None = None,
                      pixel_shuffle: int = 1, relu6_input: bool = False) -> BTensor:
        out = ctypes.c_void_p()
        check(lib().zjai_conv_forward_fused(eng.handle, self._h, x._h, act, res,
                                            r1._h if r1 else None, r2._h if r2 else None,
                                            pixel_shuffle, 1 if relu6_input else 0,
                                            ctypes.byref(out)), eng.handle)
        return BTensor(eng, out)

    def __del__(self):
        try:
            if self._h:
                lib().zjai_layer_destroy(self._h)
                self._h = None
        except Exception:
            pass


class ConvLayer(_Layer):
    """``ConvLayer::new`` / ``with_extra_pad`` (src/nn/fast/layers.rs:31-70)."""

    def __init__(self, conv: Conv2d, eng: Engine, extra_pad=(0, 0, 0, 0)):
        h = ctypes.c_void_p()
        ext = (ctypes.c_int32 * 4)(*extra_pad)
        kh, kw = conv.kernel
        check(lib().zjai_conv2d_create(eng.handle, conv.in_ch, conv.out_ch, kh, kw, conv.stride,
                                       conv.pad[0], conv.pad[1], conv.groups, _fp(conv.weight),
                                       _fp(conv.bias), ext, eng.dtype, ctypes.byref(h)),
              eng.handle)
        super().__init__(eng, h)


class ConvTransposeLayer(_Layer):
    """``ConvTransposeLayer::new`` (src/nn/fast/layers.rs:136-152)."""

    def __init__(self, conv: ConvTranspose2d, eng: Engine):
        h = ctypes.c_void_p()
        check(lib().zjai_conv_transpose2d_create(eng.handle, conv.in_ch, conv.out_ch, conv.k,
                                                 conv.stride, conv.pad, conv.out_pad,
                                                 _fp(conv.weight), _fp(conv.bias), eng.dtype,
                                                 ctypes.byref(h)), eng.handle)
        super().__init__(eng, h)


# ------------------------------------------------------------ elementwise (src/nn/fast/layers.rs)
def relu(eng: Engine, x: BTensor) -> None:
    check(lib().zjai_relu(eng.handle, x._h), eng.handle)


def relu6(eng: Engine, x: BTensor) -> None:
    check(lib().zjai_relu6(eng.handle, x._h), eng.handle)


def leaky_relu(eng: Engine, x: BTensor) -> None:
    """``hyper_encoder::leaky_relu`` (src/model/hyper_encoder.rs:24-30)."""
    check(lib().zjai_leaky_relu(eng.handle, x._h), eng.handle)


def add_assign(eng: Engine, dst: BTensor, src: BTensor) -> None:
    check(lib().zjai_add_assign(eng.handle, dst._h, src._h), eng.handle)


def gate(eng: Engine, x: BTensor, mask: BTensor) -> None:
    check(lib().zjai_gate(eng.handle, x._h, mask._h), eng.handle)


def pixel_shuffle(eng: Engine, x: BTensor, r: int) -> BTensor:
    out = ctypes.c_void_p()
    check(lib().zjai_pixel_shuffle(eng.handle, x._h, r, ctypes.byref(out)), eng.handle)
    return BTensor(eng, out)


# ------------------------------------------------------------------ math (src/nn/fast/math.rs)
def sigmoid(eng: Engine, x: BTensor) -> None:
    check(lib().zjai_sigmoid(eng.handle, x._h), eng.handle)


def mul_assign(eng: Engine, a: BTensor, b: BTensor) -> None:
    check(lib().zjai_mul_assign(eng.handle, a._h, b._h), eng.handle)


def resize(eng: Engine, x, out_h: int, out_w: int, mode: str = "bicubic") -> np.ndarray:
    """``F.interpolate(x, (out_h, out_w), mode, align_corners=True)`` on the device, as the
    reference's ``decoder::output::resize_bicubic`` (src/decoder/output.rs:117) / ``nn::resize_bilinear``
    (src/nn/resample.rs:43) compute it; x is planar [c][h][w] float32."""
    x = _f32(x)
    c, h, w = x.shape
    y = np.empty((c, out_h, out_w), np.float32)
    m = {"bicubic": _lib.RESIZE_BICUBIC, "bilinear": _lib.RESIZE_BILINEAR}[mode]
    check(lib().zjai_resize(eng.handle, m, _fp(x), c, h, w, out_h, out_w, _fp(y)), eng.handle)
    return y


def elu_gate(eng: Engine, a: BTensor, b: BTensor) -> None:
    check(lib().zjai_elu_gate(eng.handle, a._h, b._h), eng.handle)


def layer_norm_channels(eng: Engine, x: BTensor, weight, bias) -> BTensor:
    out = ctypes.c_void_p()
    check(lib().zjai_layer_norm_channels(eng.handle, x._h, _fp(_f32(weight)), _fp(_f32(bias)),
                                         ctypes.byref(out)), eng.handle)
    return BTensor(eng, out)


def channel_attention(eng: Engine, qkv: BTensor, heads: int, temperature) -> BTensor:
    out = ctypes.c_void_p()
    t = _f32(np.ravel(temperature))
    check(lib().zjai_channel_attention(eng.handle, qkv._h, heads, _fp(t), ctypes.byref(out)),
          eng.handle)
    return BTensor(eng, out)
