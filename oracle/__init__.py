"""CPU oracle for the JPEG AI synthesis hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this package, and only as the checker. The product library (``zenjpegai_amd``) never
imports, links or calls anything here.

Layer primitives are the C++ loops in ``oracle.cpp`` (restating the reference's
``src/nn/reference.rs`` and ``src/nn/fast/math.rs``); graph-level functions live in
``oracle.graphs`` and the integer tiling geometry in ``oracle.geometry``. Tensors are numpy
float32 arrays, planar ``[c, h, w]`` like the reference's ``Tensor<f32>``.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int)
_u16p = ctypes.POINTER(ctypes.c_uint16)


def build() -> None:
    """Compile ``liboracle.so`` from ``oracle.cpp`` (gcc)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.or_conv2d.restype = ctypes.c_int
        L.or_conv2d.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p, _f32p,
                                ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                ctypes.c_int, ctypes.c_int, ctypes.c_int, _i32p, _f32p]
        L.or_conv_transpose2d.restype = ctypes.c_int
        L.or_conv_transpose2d.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p,
                                          _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_int, ctypes.c_int, _f32p]
        L.or_pixel_shuffle.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_int, _f32p]
        for name in ("or_relu", "or_relu6", "or_leaky_relu", "or_denormalize", "or_exp_slice",
                     "or_sigmoid"):
            getattr(L, name).argtypes = [_f32p, ctypes.c_long]
        for name in ("or_add", "or_gate", "or_mul", "or_elu_gate"):
            getattr(L, name).argtypes = [_f32p, _f32p, ctypes.c_long]
        L.or_exp.restype = ctypes.c_float
        L.or_exp.argtypes = [ctypes.c_float]
        L.or_layer_norm_channels.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                             _f32p, _f32p]
        L.or_dot8.restype = ctypes.c_double
        L.or_dot8.argtypes = [_f32p, _f32p, ctypes.c_long]
        L.or_channel_attention.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                           ctypes.c_int, _f32p, _f32p, _f32p]
        L.or_quantize_plane.argtypes = [_f32p, ctypes.c_long, ctypes.c_int, _u16p]
        L.or_f32_to_f16.restype = ctypes.c_uint16
        L.or_f32_to_f16.argtypes = [ctypes.c_float]
        L.or_f16_to_f32.restype = ctypes.c_float
        L.or_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.or_f16_round_trip.argtypes = [_f32p, ctypes.c_long, _f32p]
        L.fc_conv2d.restype = ctypes.c_int
        L.fc_conv2d.argtypes = L.or_conv2d.argtypes
        L.fc_conv_transpose2d.restype = ctypes.c_int
        L.fc_conv_transpose2d.argtypes = L.or_conv_transpose2d.argtypes
        L.fc_block_size.restype = ctypes.c_int
        L.fc_threads.restype = ctypes.c_int
        L.fc_force_tier.restype = ctypes.c_int
        L.fc_force_tier.argtypes = [ctypes.c_int]
        L.fc_set_threads.restype = ctypes.c_int
        L.fc_set_threads.argtypes = [ctypes.c_int]
        for name in ("or_resize_bicubic", "or_resize_bilinear"):
            getattr(L, name).argtypes = [_f32p] + [ctypes.c_int] * 5 + [_f32p]
            getattr(L, name).restype = ctypes.c_int
        L.or_yuv_to_rgb.argtypes = [_f32p, _f32p, _f32p, ctypes.c_long, _f32p, _f32p, _f32p]
        L.or_quantize_rgb.argtypes = [_f32p, _f32p, _f32p, ctypes.c_long, ctypes.c_int, _u16p]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_f32p)


def _c(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


class OracleError(ValueError):
    pass


def conv2d(x, weight, bias, stride=1, pad=(0, 0), groups=1, extra_pad=(0, 0, 0, 0), fast=False):
    """``reference::conv2d`` (src/nn/reference.rs:103-133) with the optional
    ``ConvLayer::with_extra_pad`` border (src/nn/fast/layers.rs:36). ``fast=True`` runs the
    restated ``nn::fast`` blocked engine (``fast_cpu.cpp``) instead: same result, bit for bit."""
    x, weight = _c(x), _c(weight)
    c, h, w = x.shape
    out_ch, _icg, kh, kw = weight.shape
    ih, iw = h + extra_pad[0] + extra_pad[2], w + extra_pad[1] + extra_pad[3]
    oh = (ih + 2 * pad[0] - kh) // stride + 1
    ow = (iw + 2 * pad[1] - kw) // stride + 1
    y = np.empty((out_ch, oh, ow), np.float32)
    b = _c(bias) if bias is not None else None
    ext = (ctypes.c_int * 4)(*extra_pad)
    fn = lib().fc_conv2d if fast else lib().or_conv2d
    rc = fn(_p(x), c, h, w, _p(weight), _p(b) if b is not None else None, out_ch,
            kh, kw, stride, pad[0], pad[1], groups, ext, _p(y))
    if rc:
        raise OracleError("conv2d: inconsistent geometry")
    return y


def conv_transpose2d(x, weight, bias, stride, pad, out_pad, fast=False):
    """``reference::conv_transpose2d`` (src/nn/reference.rs:206-236); weight [in][out][k][k].
    ``fast=True``: the restated ``nn::fast`` phase driver (stride 2, k <= 4), same result."""
    x, weight = _c(x), _c(weight)
    c, h, w = x.shape
    _, out_ch, k, _ = weight.shape
    oh = (h - 1) * stride + k + out_pad - 2 * pad
    ow = (w - 1) * stride + k + out_pad - 2 * pad
    y = np.empty((out_ch, oh, ow), np.float32)
    b = _c(bias) if bias is not None else None
    fn = lib().fc_conv_transpose2d if fast else lib().or_conv_transpose2d
    rc = fn(_p(x), c, h, w, _p(weight), _p(b) if b is not None else None,
            out_ch, k, stride, pad, out_pad, _p(y))
    if rc:
        raise OracleError("conv_transpose2d: unsupported geometry")
    return y


def pixel_shuffle(x, r):
    x = _c(x)
    c, h, w = x.shape
    if c % (r * r):
        raise OracleError("pixel_shuffle: channels not divisible by r^2")
    y = np.empty((c // (r * r), h * r, w * r), np.float32)
    lib().or_pixel_shuffle(_p(x), c, h, w, r, _p(y))
    return y


def _unary(name, x):
    y = _c(x).copy()
    getattr(lib(), name)(_p(y), y.size)
    return y


def _binary(name, a, b):
    y = _c(a).copy()
    b = _c(b)
    assert b.shape == y.shape
    getattr(lib(), name)(_p(y), _p(b), y.size)
    return y


def relu(x):
    return _unary("or_relu", x)


def relu6(x):
    return _unary("or_relu6", x)


def leaky_relu(x):
    return _unary("or_leaky_relu", x)


def denormalize(x):
    return _unary("or_denormalize", x)


def exp(x):
    return _unary("or_exp_slice", x)


def sigmoid(x):
    return _unary("or_sigmoid", x)


def add(a, b):
    return _binary("or_add", a, b)


def gate(x, mask):
    """``x * (1 + mask)`` (src/nn/fast/layers.rs:195-201)."""
    return _binary("or_gate", x, mask)


def mul(a, b):
    return _binary("or_mul", a, b)


def elu_gate(a, b):
    return _binary("or_elu_gate", a, b)


def layer_norm_channels(x, weight, bias):
    y = _c(x).copy()
    c, h, w = y.shape
    lib().or_layer_norm_channels(_p(y), c, h, w, _p(_c(weight)), _p(_c(bias)))
    return y


def dot8(a, b):
    a, b = _c(a).ravel(), _c(b).ravel()
    return lib().or_dot8(_p(a), _p(b), a.size)


def channel_attention(qkv, heads, temperature, return_attn=False):
    qkv = _c(qkv)
    c3, h, w = qkv.shape
    dim = c3 // 3
    out = np.empty((dim, h, w), np.float32)
    attn = np.empty((dim, dim // heads), np.float32)
    rc = lib().or_channel_attention(_p(qkv), c3, h, w, heads, _p(_c(temperature)), _p(out),
                                    _p(attn))
    if rc:
        raise OracleError("attention: channel / head counts")
    return (out, attn) if return_attn else out


def quantize_plane(x, bit_depth):
    x = _c(x)
    out = np.empty(x.shape, np.uint16)
    lib().or_quantize_plane(_p(x), x.size, bit_depth, out.ctypes.data_as(_u16p))
    return out


def resize_bicubic(x, oh, ow):
    """``F.interpolate(x, (oh, ow), mode="bicubic", align_corners=True)`` as the reference's
    ``decoder::output::resize_bicubic`` (src/decoder/output.rs:100-147) computes it; x is
    [c][h][w]."""
    x = _c(x)
    c, h, w = x.shape
    y = np.empty((c, oh, ow), np.float32)
    if lib().or_resize_bicubic(_p(x), c, h, w, oh, ow, _p(y)):
        raise ValueError("resize: empty input")
    return y


def resize_bilinear(x, oh, ow):
    """``nn::resize_bilinear`` (src/nn/resample.rs:43-69), align_corners; x is [c][h][w]."""
    x = _c(x)
    c, h, w = x.shape
    y = np.empty((c, oh, ow), np.float32)
    if lib().or_resize_bilinear(_p(x), c, h, w, oh, ow, _p(y)):
        raise ValueError("resize: empty dimension")
    return y


def yuv_to_rgb(y, u, v):
    """BT.709 4:4:4 planes in [0, 255] -> clipped RGB planes (src/decoder/output.rs:232-257)."""
    y, u, v = _c(y), _c(u), _c(v)
    assert y.shape == u.shape == v.shape
    r, g, b = (np.empty(y.shape, np.float32) for _ in range(3))
    lib().or_yuv_to_rgb(_p(y), _p(u), _p(v), y.size, _p(r), _p(g), _p(b))
    return r, g, b


def quantize_rgb(r, g, b, bit_depth):
    """Interleaved [h][w][3] uint16 RGB samples (src/decoder/output.rs:407-437)."""
    r, g, b = _c(r), _c(g), _c(b)
    out = np.empty(r.shape + (3,), np.uint16)
    lib().or_quantize_rgb(_p(r), _p(g), _p(b), r.size, bit_depth, out.ctypes.data_as(_u16p))
    return out


def picture_rgb(y, u, v, bit_depth):
    """`finish` for a BT.709 stream (src/decoder/output.rs:346-366) after `to_source_format`
    (:153-199): chroma planes of any coded subsampling are bicubic-resampled to the luma size,
    converted and quantised. Returns (interleaved uint16 RGB, float RGB planes)."""
    y = _c(y)
    h, w = y.shape
    u = _c(u)[None]
    v = _c(v)[None]
    if u.shape[1:] != (h, w):
        u = resize_bicubic(u, h, w)
        v = resize_bicubic(v, h, w)
    r, g, b = yuv_to_rgb(y, u[0], v[0])
    return quantize_rgb(r, g, b, bit_depth), np.stack([r, g, b])


def f32_to_f16_bits(v: float) -> int:
    return lib().or_f32_to_f16(v)


def f16_bits_to_f32(h: int) -> float:
    return lib().or_f16_to_f32(h)


def f16_round_trip(x):
    x = _c(x)
    y = np.empty_like(x)
    lib().or_f16_round_trip(_p(x), x.size, _p(y))
    return y


def force_cpu_tier(v: int) -> None:
    """Pins the ``nn::fast`` restatement to its AVX2 (8) or AVX-512 (16) tier; 0 = automatic."""
    if lib().fc_force_tier(v):
        raise OracleError(f"CPU tier {v} is not available on this host")


def set_cpu_threads(n: int) -> None:
    """Sets the OpenMP threads of the CPU restatements (``fast_cpu.cpp`` and ``oracle.cpp``)."""
    if lib().fc_set_threads(int(n)):
        raise OracleError(f"thread count {n}")


def cpu_threads() -> int:
    return lib().fc_threads()
