"""ctypes binding of ``libzjai_hip.so`` (the C-ABI declared in ``include/zjai_hip.h``).

The library is built in-tree (``make -C zenjpegai_amd/csrc`` or ``__graft_entry__.build()``).
There is no fallback: if the library is missing or cannot be loaded, :func:`lib` raises.
"""

from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libzjai_hip.so")

OK = 0
E_INVALID_ARGUMENT = -1
E_UNSUPPORTED = -2
E_LIMIT = -3
E_MODEL = -4
E_CANCELLED = -5
E_DEVICE = -6
ERROR_NAMES = {
    E_INVALID_ARGUMENT: "InvalidArgument",
    E_UNSUPPORTED: "Unsupported",
    E_LIMIT: "LimitExceeded",
    E_MODEL: "Model",
    E_CANCELLED: "Cancelled",
    E_DEVICE: "Device",
}

F32, F16, BF16 = 0, 1, 2
PRECISIONS = {"f32": F32, "f16": F16, "bf16": BF16}
OPS = {"sop": 0, "bop": 1, "hop": 2}
ACT_NONE, ACT_RELU, ACT_LEAKY_RELU, ACT_SIGMOID = 0, 1, 2, 3
RES_NONE, RES_ADD, RES_GATE, RES_CAB, RES_MUL = 0, 1, 2, 3, 4
CTX_UNFUSED_BLOCKS = 0x1  # zjai_ctx_create flags
CTX_PHASE_SPLIT_CONVT = 0x2
CTX_MFMA16_CONV3X3 = 0x4
CTX_IGEMM_CONV1X1 = 0x8
CTX_COUNT_F16_RANGE = 0x10
CTX_VALU_NARROW_CONVT = 0x20
FAIL_NONE, FAIL_ALLOC, FAIL_LAUNCH = 0, 1, 2  # zjai_inject_failure kinds
RESIZE_BICUBIC, RESIZE_BILINEAR = 0, 1
PLANE_LATENT, PLANE_PSI, PLANE_HYPER_LATENT, PLANE_IMAGE = 0, 1, 2, 3


class ZjaiTile(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "image_x", "image_y", "image_w", "image_h", "latent_x", "latent_y", "latent_w",
        "latent_h", "core_x", "core_y", "core_w", "core_h", "core_off_x", "core_off_y")]


class ZjaiRegions(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "num_ver", "num_hor", "independent", "hyper_decoder_overlap", "mcm_overlap")]


class ZjaiArea(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("x", "y", "width", "height")]


class ZjaiStats(ctypes.Structure):
    _fields_ = [("last_run_ms", ctypes.c_float), ("kernel_launches", ctypes.c_int64),
                ("pool_in_use", ctypes.c_uint64), ("pool_peak", ctypes.c_uint64),
                ("pool_cached", ctypes.c_uint64), ("f16_nonfinite", ctypes.c_uint64)]


class ZjaiMemoryEstimate(ctypes.Structure):
    _fields_ = [("picture_bytes", ctypes.c_uint64), ("live_bytes", ctypes.c_uint64),
                ("pool_bytes", ctypes.c_uint64)]


class ZjaiProfRecord(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 96), ("flops", ctypes.c_double),
                ("bytes", ctypes.c_double), ("ms", ctypes.c_float)]


_vp = ctypes.c_void_p
_pp = ctypes.POINTER(ctypes.c_void_p)
_i32 = ctypes.c_int32
_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)
_sz = ctypes.c_size_t

# name -> argtypes (every entry point returns int32)
PROTOTYPES = {
    "zjai_ctx_create": [_i32, ctypes.c_uint32, _pp],
    "zjai_ctx_destroy": [_vp],
    "zjai_last_error": [_vp, ctypes.c_char_p, ctypes.c_size_t],
    "zjai_sync": [_vp],
    "zjai_set_stop": [_vp, _i32],
    "zjai_get_stats": [_vp, ctypes.POINTER(ZjaiStats)],
    "zjai_release_buffers": [_vp],
    "zjai_inject_failure": [_vp, _i32, ctypes.c_int64],
    "zjai_profile_begin": [_vp],
    "zjai_profile_end": [_vp, ctypes.POINTER(ZjaiProfRecord), _i32, _i32p],
    "zjai_tensor_create": [_vp, _i32, _i32, _i32, _i32, _pp],
    "zjai_tensor_from_planar": [_vp, _f32p, _i32, _i32, _i32, _i32, _pp],
    "zjai_tensor_to_planar": [_vp, _vp, _f32p, ctypes.c_size_t],
    "zjai_tensor_shape": [_vp, _i32p, _i32p, _i32p, _i32p],
    "zjai_tensor_crop": [_vp, _vp, _i32, _i32, _pp],
    "zjai_tensor_cat": [_vp, _pp, _i32, _pp],
    "zjai_tensor_destroy": [_vp],
    "zjai_conv2d_create": [_vp, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32p, _f32p,
                           _i32p, _i32, _pp],
    "zjai_conv_transpose2d_create": [_vp, _i32, _i32, _i32, _i32, _i32, _i32, _f32p, _f32p,
                                     _i32, _pp],
    "zjai_layer_destroy": [_vp],
    "zjai_conv_forward": [_vp, _vp, _vp, _pp],
    "zjai_conv_forward_fused": [_vp, _vp, _vp, _i32, _i32, _vp, _vp, _i32, _i32, _pp],
    "zjai_relu": [_vp, _vp],
    "zjai_relu6": [_vp, _vp],
    "zjai_leaky_relu": [_vp, _vp],
    "zjai_sigmoid": [_vp, _vp],
    "zjai_add_assign": [_vp, _vp, _vp],
    "zjai_gate": [_vp, _vp, _vp],
    "zjai_mul_assign": [_vp, _vp, _vp],
    "zjai_elu_gate": [_vp, _vp, _vp],
    "zjai_pixel_shuffle": [_vp, _vp, _i32, _pp],
    "zjai_layer_norm_channels": [_vp, _vp, _f32p, _f32p, _pp],
    "zjai_channel_attention": [_vp, _vp, _i32, _f32p, _pp],
    "zjai_channel_attention_noalloc": [_vp, _vp, _i32, _i32, _i32, _i32, _vp, _i32, _vp],
    "zjai_net_create": [_vp, _i32, _i32, _i32, _i32, ctypes.POINTER(ctypes.c_char_p), _i32p,
                        _i32p, ctypes.POINTER(_f32p), _pp],
    "zjai_net_destroy": [_vp],
    "zjai_net_out_size": [_vp, _i32, _i32, _i32p, _i32p],
    "zjai_net_device_bytes": [_vp, ctypes.POINTER(ctypes.c_uint64)],
    "zjai_primary_forward": [_vp, _vp, _vp, _i32, _i32, _f32p, ctypes.c_size_t],
    "zjai_secondary_forward": [_vp, _vp, _vp, _vp, _i32, _i32, _f32p, ctypes.c_size_t],
    "zjai_synthesis_tiles": [_i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                             ctypes.POINTER(ZjaiTile), _i32, _i32p],
    "zjai_picture_create": [_vp, _vp, _vp, _i32, _i32, _i32, _i32, ctypes.POINTER(ZjaiTile),
                            _i32, _i32, _i32, _i32, _i32, _i32, _pp],
    "zjai_picture_destroy": [_vp],
    "zjai_picture_estimate_memory": [_i32, _i32, _i32, _i32, _i32, _i32, _i32,
                                     ctypes.POINTER(ZjaiTile), _i32, _i32, _i32, _i32, _i32, _i32,
                                     _i32, ctypes.POINTER(ZjaiMemoryEstimate)],
    "zjai_ctx_set_memory_limit": [_vp, ctypes.c_uint64],
    "zjai_picture_upload": [_vp, _vp, _f32p, _f32p],
    "zjai_picture_run": [_vp, _vp],
    "zjai_picture_set_lanes": [_vp, _vp, _i32],
    "zjai_picture_set_replay": [_vp, _vp, _i32],
    "zjai_picture_download": [_vp, _vp, _vp, _vp, _vp],
    "zjai_host_alloc": [_vp, _sz, _pp],
    "zjai_host_free": [_vp, _vp],
    "zjai_resize": [_vp, _i32, _f32p, _i32, _i32, _i32, _i32, _i32, _f32p],
    "zjai_picture_download_rgb": [_vp, _vp, _i32, _vp, _f32p],
    "zjai_region_grid": [_i32, _i32, _i32, ctypes.POINTER(ZjaiRegions), _i32,
                         ctypes.POINTER(ZjaiArea), ctypes.POINTER(ZjaiArea), _i32, _i32p],
    "zjai_latent_model_create": [_vp, _i32, _i32, _i32, ctypes.POINTER(ctypes.c_char_p), _i32p,
                                 _i32p, ctypes.POINTER(_f32p), _pp],
    "zjai_latent_model_info": [_vp, _i32p, _i32p],
    "zjai_hyper_decoder_forward": [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _f32p,
                                   ctypes.c_size_t],
    "zjai_context_decompress": [_vp, _vp, _f32p, _i32, _i32, _i32, _f32p, _i32, _i32, _f32p,
                                ctypes.c_size_t],
    "zjai_reconstruct_latent": [_vp, _vp, _i32, _i32, ctypes.POINTER(ZjaiRegions), _vp, _i32,
                                _i32, _f32p, _i32, _i32, _f32p, _f32p],
    # weight readers (host only)
    "zjai_checkpoint_parse": [_vp, _sz, _pp],
    "zjai_checkpoint_destroy": [_vp],
    "zjai_checkpoint_counts": [_vp, _i32p, _i32p, _i32p, _i32p],
    "zjai_checkpoint_tensor_name": [_vp, _i32, ctypes.c_char_p, _sz],
    "zjai_checkpoint_info": [_vp, ctypes.c_char_p, _i32p, _i32p, ctypes.POINTER(ctypes.c_int64)],
    "zjai_checkpoint_read": [_vp, ctypes.c_char_p, _vp, _sz],
    "zjai_checkpoint_read_f32": [_vp, ctypes.c_char_p, _f32p, _sz],
    "zjai_checkpoint_int_at": [_vp, _i32, ctypes.c_char_p, _sz, ctypes.POINTER(ctypes.c_int64)],
    "zjai_checkpoint_list_at": [_vp, _i32, ctypes.c_char_p, _sz, ctypes.POINTER(ctypes.c_double),
                                _sz, ctypes.POINTER(_sz)],
    "zjai_checkpoint_write_zjm": [_vp, ctypes.POINTER(ctypes.c_char_p), _i32, _i32, _vp, _sz,
                                  ctypes.POINTER(_sz)],
    "zjai_bundle_parse": [_vp, _sz, _pp],
    "zjai_bundle_add": [_vp, _vp, _sz],
    "zjai_bundle_destroy": [_vp],
    "zjai_bundle_count": [_vp, _i32p],
    "zjai_bundle_path": [_vp, _i32, ctypes.c_char_p, _sz],
    "zjai_bundle_get": [_vp, ctypes.c_char_p, _pp, ctypes.POINTER(_sz)],
    "zjai_bundle_notice": [_vp, ctypes.c_char_p, _sz, ctypes.POINTER(_sz)],
    "zjai_bundle_write": [ctypes.POINTER(ctypes.c_char_p), _pp, ctypes.POINTER(_sz), _i32,
                          ctypes.c_char_p, _i32, _vp, _sz, ctypes.POINTER(_sz)],
    "zjai_net_create_from_checkpoint": [_vp, _i32, _i32, _i32, _vp, _pp],
    "zjai_latent_model_create_from_checkpoint": [_vp, _i32, _i32, _vp, _pp],
    "zjai_analysis_create": [_vp, _i32, _i32, _i32, _i32, ctypes.POINTER(ctypes.c_char_p), _i32p,
                             _i32p, ctypes.POINTER(_f32p), _pp],
    "zjai_analysis_create_from_checkpoint": [_vp, _i32, _i32, _i32, _vp, _pp],
    "zjai_analysis_forward": [_vp, _vp, _f32p, _i32, _i32, _i32, _i32, _f32p, _sz],
}

_lib = None


class HipError(RuntimeError):
    """A failed C-ABI call: ``code`` is the ZJAI_E_* status, ``kind`` its reference
    ``zenjpegai::Error`` variant name."""

    def __init__(self, code: int, message: str):
        self.code = code
        self.kind = ERROR_NAMES.get(code, f"code {code}")
        super().__init__(f"{self.kind}: {message}")


def lib():
    """Loads the HIP library; raises if it is missing (no CPU fallback exists)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build()")
        L = ctypes.CDLL(LIB_PATH)
        for name, args in PROTOTYPES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int32
        _lib = L
    return _lib


def last_error(ctx) -> str:
    buf = ctypes.create_string_buffer(1024)
    lib().zjai_last_error(ctx, buf, len(buf))
    return buf.value.decode(errors="replace")


def check(rc: int, ctx=None) -> None:
    if rc != OK:
        raise HipError(rc, last_error(ctx))
