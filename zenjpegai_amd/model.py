"""Graph-level surface: the synthesis transforms (``src/model/synthesis.rs``) and the picture
driver (``src/decoder/reconstruct.rs`` synthesis half + ``quantize_plane``), over the C-ABI."""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import HipError, check, lib
from .nn import BTensor, Engine, _f32, _fp
from .weights import Checkpoint


def _descriptors(params: dict):
    """(n, names, ndims, dims, data pointers, arrays kept alive) of named checkpoint tensors."""
    names, ndims, dims, ptrs, keep = [], [], [], [], []
    for name, arr in params.items():
        a = _f32(arr)
        keep.append(a)
        names.append(name.encode())
        ndims.append(a.ndim)
        dims.extend(a.shape)
        ptrs.append(a.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    n = len(names)
    c_names = (ctypes.c_char_p * n)(*names)
    c_ndims = (ctypes.c_int32 * n)(*ndims)
    c_dims = (ctypes.c_int32 * max(len(dims), 1))(*dims)
    c_ptrs = (ctypes.POINTER(ctypes.c_float) * n)(*ptrs)
    return n, c_names, c_ndims, c_dims, c_ptrs, keep


def _net_create(eng: Engine, op: str, component: int, params):
    h = ctypes.c_void_p()
    if isinstance(params, Checkpoint):
        check(lib().zjai_net_create_from_checkpoint(eng.handle, _lib.OPS[op], component, eng.dtype,
                                                    params.handle, ctypes.byref(h)), eng.handle)
        return h
    n, c_names, c_ndims, c_dims, c_ptrs, _keep = _descriptors(params)
    check(lib().zjai_net_create(eng.handle, _lib.OPS[op], component, eng.dtype, n, c_names,
                                c_ndims, c_dims, c_ptrs, ctypes.byref(h)), eng.handle)
    return h


class _Net:
    component = 0

    def __init__(self, eng: Engine, params: dict, op: str):
        self.eng = eng
        self.op = op
        self._h = _net_create(eng, op, self.component, params)

    @classmethod
    def load(cls, params: dict, op: str, eng: Engine):
        """``SynthesisPrimary::load(ck, op, eng)`` / ``SynthesisSecondary::load``: ``params``
        is a ``weights.Checkpoint`` or maps checkpoint names to arrays."""
        return cls(eng, params, op)

    def out_size(self, h: int, w: int):
        oh, ow = ctypes.c_int32(), ctypes.c_int32()
        check(lib().zjai_net_out_size(self._h, h, w, ctypes.byref(oh), ctypes.byref(ow)),
              self.eng.handle)
        return oh.value, ow.value

    def device_bytes(self) -> int:
        """Device bytes of the net's packed weights, biases and vectors."""
        n = ctypes.c_uint64()
        check(lib().zjai_net_device_bytes(self._h, ctypes.byref(n)), self.eng.handle)
        return n.value

    def __del__(self):
        try:
            if self._h:
                lib().zjai_net_destroy(self._h)
                self._h = None
        except Exception:
            pass


class SynthesisPrimary(_Net):
    """Luma synthesis (``SynthesisPrimary``, src/model/synthesis.rs:233-312)."""
    component = 0

    def forward(self, eng: Engine, y_hat: BTensor, h: int, w: int) -> np.ndarray:
        """``y_hat [160, H, W]`` -> ``[1, >=h, >=w]`` in [0, 255] (the caller crops)."""
        oh, ow = self.out_size(h, w)
        out = np.empty((1, oh, ow), np.float32)
        check(lib().zjai_primary_forward(eng.handle, self._h, y_hat._h, h, w, _fp(out),
                                         out.size), eng.handle)
        return out


class SynthesisSecondary(_Net):
    """Chroma synthesis (``SynthesisSecondary``, src/model/synthesis.rs:709-1038)."""
    component = 1

    def forward(self, eng: Engine, y_hat_luma: BTensor, y_hat_chroma: BTensor, h: int,
                w: int) -> np.ndarray:
        oh, ow = self.out_size(h, w)
        out = np.empty((2, oh, ow), np.float32)
        check(lib().zjai_secondary_forward(eng.handle, self._h, y_hat_luma._h, y_hat_chroma._h,
                                           h, w, _fp(out), out.size), eng.handle)
        return out


@dataclass(frozen=True)
class Area:
    x: int
    y: int
    width: int
    height: int


@dataclass(frozen=True)
class SynthesisTile:
    """``tools::tiles::SynthesisTile`` (src/tools/tiles.rs:26-35)."""
    image: Area
    latent: Area
    core: Area
    core_offset: tuple


def synthesis_tiles(height, width, latent_h, latent_w, tiling=None, region_grid=None):
    """``synthesis_tiles`` (src/tools/tiles.rs:39-119) computed by the library. ``tiling`` is
    ``(tile_size, overlap)`` or None; ``region_grid`` is ``(rows, cols)`` of independent regions
    or None."""
    size, overlap = tiling if tiling else (0, 0)
    rows, cols = region_grid if region_grid else (0, 0)
    cap = 4096
    buf = (_lib.ZjaiTile * cap)()
    n = ctypes.c_int32()
    check(lib().zjai_synthesis_tiles(height, width, latent_h, latent_w, size, overlap, rows, cols,
                                     buf, cap, ctypes.byref(n)), None)
    out = []
    for t in buf[:n.value]:
        out.append(SynthesisTile(Area(t.image_x, t.image_y, t.image_w, t.image_h),
                                 Area(t.latent_x, t.latent_y, t.latent_w, t.latent_h),
                                 Area(t.core_x, t.core_y, t.core_w, t.core_h),
                                 (t.core_off_x, t.core_off_y)))
    return out


def _tile_array(tiles):
    arr = (_lib.ZjaiTile * len(tiles))()
    for i, t in enumerate(tiles):
        arr[i] = _lib.ZjaiTile(t.image.x, t.image.y, t.image.width, t.image.height,
                               t.latent.x, t.latent.y, t.latent.width, t.latent.height,
                               t.core.x, t.core.y, t.core.width, t.core.height,
                               t.core_offset[0], t.core_offset[1])
    return arr


def estimate_picture_memory(op: str, precision: str, with_uv: bool, lh: int, lw: int, height: int,
                            width: int, tiles, sv: int = 1, sh: int = 1, out_h: int | None = None,
                            out_w: int | None = None, bit_depth: int = 0, lanes: int = 1) -> dict:
    """Device bytes of a picture before it is created (``estimate_memory``,
    src/decoder/limits.rs:164-245; ``zjai_picture_estimate_memory``, host only):
    ``picture_bytes`` (latents and planes, exact), ``live_bytes`` (the tile batches' buffer-pool
    blocks in use at once over all lanes) and ``pool_bytes`` (the blocks the pools keep after the
    run), both modelled from above. The nets' bytes (``device_bytes()``) come on top."""
    arr = _tile_array(list(tiles))
    e = _lib.ZjaiMemoryEstimate()
    check(lib().zjai_picture_estimate_memory(
        _lib.OPS[op], _lib.PRECISIONS[precision], 1 if with_uv else 0, lh, lw, height, width, arr,
        len(arr), sv, sh, height if out_h is None else out_h, width if out_w is None else out_w,
        bit_depth, lanes, ctypes.byref(e)), None)
    return {k: getattr(e, k) for k, _ in e._fields_}


class Picture:
    """A planned whole-picture synthesis: latents uploaded once, tile batches on one stream or
    on `lanes` concurrent streams (``zjai_picture_set_lanes``), tile cores written (and
    quantised) straight into the output planes."""

    def __init__(self, eng: Engine, primary: SynthesisPrimary,
                 secondary: SynthesisSecondary | None, lh: int, lw: int, height: int,
                 width: int, tiles, sv: int = 1, sh: int = 1, out_h: int | None = None,
                 out_w: int | None = None, bit_depth: int = 0, lanes: int = 1):
        self.eng = eng
        self.primary, self.secondary = primary, secondary
        self.lh, self.lw, self.height, self.width = lh, lw, height, width
        self.sv, self.sh, self.bit_depth = sv, sh, bit_depth
        self.out_h = height if out_h is None else out_h
        self.out_w = width if out_w is None else out_w
        self.tiles = list(tiles)
        self._tiles = _tile_array(self.tiles)
        self._h = ctypes.c_void_p()
        check(lib().zjai_picture_create(eng.handle, primary._h, secondary._h if secondary else None,
                                        lh, lw, height, width, self._tiles, len(self.tiles), sv,
                                        sh, self.out_h, self.out_w, bit_depth,
                                        ctypes.byref(self._h)), eng.handle)
        self.set_lanes(lanes)

    def set_lanes(self, lanes: int):
        check(lib().zjai_picture_set_lanes(self.eng.handle, self._h, lanes), self.eng.handle)
        self.lanes = lanes

    def set_replay(self, on: bool):
        """Replay mode: the next run captures the whole launch sequence as a HIP graph, later
        runs replay it (``zjai_picture_set_replay``)."""
        check(lib().zjai_picture_set_replay(self.eng.handle, self._h, 1 if on else 0), self.eng.handle)

    def upload(self, y_hat: np.ndarray, uv_hat: np.ndarray | None = None):
        self._y = _f32(y_hat)
        self._uv = _f32(uv_hat)
        assert self._y.shape == (160, self.lh, self.lw)
        check(lib().zjai_picture_upload(self.eng.handle, self._h, _fp(self._y), _fp(self._uv)),
              self.eng.handle)

    def run(self):
        check(lib().zjai_picture_run(self.eng.handle, self._h), self.eng.handle)

    def download(self, out=None):
        """The Y, U, V planes (U, V None without a chroma net); ``out``: preallocated (y, u, v)
        arrays of the right shapes and dtype to fill instead, e.g. from ``Engine.host_array``."""
        dt = np.uint16 if self.bit_depth else np.float32
        ch, cw = -(-self.out_h // self.sv), -(-self.out_w // self.sh)
        if out is not None:
            y, u, v = out
            want = [(y, (self.out_h, self.out_w))] + ([(u, (ch, cw)), (v, (ch, cw))] if self.secondary else [])
            for a, shape in want:
                if a is None or a.shape != shape or a.dtype != dt or not a.flags.c_contiguous:
                    raise HipError(_lib.E_INVALID_ARGUMENT, "download: output arrays of the wrong shape or dtype")
            if not self.secondary:
                u = v = None
        else:
            y = np.empty((self.out_h, self.out_w), dt)
            u = np.empty((ch, cw), dt) if self.secondary else None
            v = np.empty((ch, cw), dt) if self.secondary else None
        check(lib().zjai_picture_download(
            self.eng.handle, self._h, y.ctypes.data_as(ctypes.c_void_p),
            u.ctypes.data_as(ctypes.c_void_p) if u is not None else None,
            v.ctypes.data_as(ctypes.c_void_p) if v is not None else None), self.eng.handle)
        return y, u, v

    def download_rgb(self, bit_depth=8, planes=False):
        """The output stage of a BT.709 stream on the device (``to_source_format`` then
        ``finish``, src/decoder/output.rs:153-199, :346-366): interleaved uint16 RGB
        [out_h][out_w][3], plus the float RGB planes [3][out_h][out_w] when ``planes``. The
        picture must have float planes (bit_depth 0) and a chroma net."""
        rgb = np.empty((self.out_h, self.out_w, 3), np.uint16)
        f = np.empty((3, self.out_h, self.out_w), np.float32) if planes else None
        check(lib().zjai_picture_download_rgb(
            self.eng.handle, self._h, bit_depth, rgb.ctypes.data_as(ctypes.c_void_p),
            f.ctypes.data_as(ctypes.POINTER(ctypes.c_float)) if planes else None), self.eng.handle)
        return (rgb, f) if planes else rgb

    def __del__(self):
        try:
            if self._h:
                lib().zjai_picture_destroy(self._h)
                self._h = None
        except Exception:
            pass


def synthesize(eng: Engine, primary, secondary, y_hat, uv_hat, height, width, tiles, sv=1, sh=1,
               out_h=None, out_w=None, bit_depth=0, lanes=1):
    """``reconstruct::synthesize_with`` (src/decoder/reconstruct.rs:285-331) followed by
    ``quantize_plane`` when ``bit_depth`` > 0: returns ``(rec_y, rec_u, rec_v)``."""
    lh, lw = y_hat.shape[1:]
    pic = Picture(eng, primary, secondary, lh, lw, height, width, tiles, sv, sh, out_h, out_w,
                  bit_depth, lanes)
    pic.upload(y_hat, uv_hat)
    pic.run()
    return pic.download()


# ---------------------------------------------------------------------------------------------
# Latent reconstruction (src/decoder/reconstruct.rs:81-234)
# ---------------------------------------------------------------------------------------------

@dataclass(frozen=True)
class Regions:
    """Region partitioning of a picture header (``Regions``, src/header.rs): region rows and
    columns, independence and the signalled overlaps (hyper-decoder x2, context model x4)."""
    num_ver: int
    num_hor: int
    independent: bool = True
    hyper_decoder_overlap: int = 0
    mcm_overlap: int = 0

    def _c(self):
        return _lib.ZjaiRegions(self.num_ver, self.num_hor, int(self.independent),
                                self.hyper_decoder_overlap, self.mcm_overlap)


PLANES = {"latent": _lib.PLANE_LATENT, "psi": _lib.PLANE_PSI,
          "hyper_latent": _lib.PLANE_HYPER_LATENT, "image": _lib.PLANE_IMAGE}


def _regions_ptr(regions):
    if regions is None:
        return None, None
    r = regions._c()
    return r, ctypes.byref(r)


def region_grid(height: int, width: int, ccs: int, regions: Regions | None, plane: str):
    """``region_grid(hdr, ccs, plane)`` (src/tools/regions.rs:116-150): ``(core, extended)``,
    lists of ``Area`` in row-major region order. ``regions=None``: not partitioned."""
    cap = 64
    core = (_lib.ZjaiArea * cap)()
    ext = (_lib.ZjaiArea * cap)()
    n = ctypes.c_int32()
    _keep, rp = _regions_ptr(regions)
    check(lib().zjai_region_grid(height, width, ccs, rp, PLANES[plane], core, ext, cap,
                                 ctypes.byref(n)))
    conv = lambda a: Area(a.x, a.y, a.width, a.height)  # noqa: E731
    return [conv(core[i]) for i in range(n.value)], [conv(ext[i]) for i in range(n.value)]


class LatentModel:
    """The float half of ``CommonModel`` (src/model/common.rs:117-129) for one component: the
    ``HyperDecoder`` and, when the checkpoint holds one, the multi-stage ``ContextModel``."""

    def __init__(self, eng: Engine, params: dict, component: int):
        self.eng = eng
        self.component = component
        self._h = ctypes.c_void_p()
        if isinstance(params, Checkpoint):
            check(lib().zjai_latent_model_create_from_checkpoint(
                eng.handle, component, eng.dtype, params.handle, ctypes.byref(self._h)), eng.handle)
        else:
            n, c_names, c_ndims, c_dims, c_ptrs, _keep = _descriptors(params)
            check(lib().zjai_latent_model_create(eng.handle, component, eng.dtype, n, c_names,
                                                 c_ndims, c_dims, c_ptrs, ctypes.byref(self._h)),
                  eng.handle)
        c, ctx = ctypes.c_int32(), ctypes.c_int32()
        check(lib().zjai_latent_model_info(self._h, ctypes.byref(c), ctypes.byref(ctx)))
        self.channels, self.has_context = c.value, bool(ctx.value)

    @classmethod
    def load(cls, params: dict, component: int, eng: Engine):
        return cls(eng, params, component)

    def hyper_decoder(self, z_hat: np.ndarray, out_h: int, out_w: int) -> np.ndarray:
        """``HyperDecoder::forward`` (src/model/hyper_decoder.rs:47): int8 ``[C, hz, wz]`` ->
        psi ``[4C, out_h, out_w]``."""
        z = np.ascontiguousarray(z_hat, dtype=np.int8)
        c, zh, zw = z.shape
        out = np.empty((4 * c, out_h, out_w), np.float32)
        check(lib().zjai_hyper_decoder_forward(self.eng.handle, self._h, z.ctypes.data, c, zh, zw,
                                               out_h, out_w, _fp(out), out.size), self.eng.handle)
        return out

    def decompress(self, residual: np.ndarray, psi: np.ndarray) -> np.ndarray:
        """``ContextModel::decompress`` (src/model/mcm.rs:161), or the up-shuffled psi plus the
        residual without a context model: residual ``[C, h, w]``, psi ``[4C, ceil(h/2),
        ceil(w/2)]`` -> y_hat ``[C, h, w]``."""
        r = np.ascontiguousarray(residual, dtype=np.float32)
        p = np.ascontiguousarray(psi, dtype=np.float32)
        c, h, w = r.shape
        out = np.empty_like(r)
        check(lib().zjai_context_decompress(self.eng.handle, self._h, _fp(r), c, h, w, _fp(p),
                                            p.shape[1], p.shape[2], _fp(out), out.size),
              self.eng.handle)
        return out

    def reconstruct(self, height: int, width: int, regions: Regions | None, z_hat: np.ndarray,
                    residual: np.ndarray):
        """``reconstruct_latent`` (src/decoder/reconstruct.rs:81): ``(psi, y_hat)`` of this
        component of a ``height x width`` picture."""
        z = np.ascontiguousarray(z_hat, dtype=np.int8)
        r = np.ascontiguousarray(residual, dtype=np.float32)
        c, h, w = r.shape
        psi = np.empty((4 * c, -(-h // 2), -(-w // 2)), np.float32)
        y = np.empty_like(r)
        _keep, rp = _regions_ptr(regions)
        check(lib().zjai_reconstruct_latent(self.eng.handle, self._h, height, width, rp,
                                            z.ctypes.data, z.shape[1], z.shape[2], _fp(r), h, w,
                                            _fp(psi), _fp(y)), self.eng.handle)
        return psi, y

    def __del__(self):
        try:
            if self._h:
                lib().zjai_net_destroy(self._h)
                self._h = None
        except Exception:
            pass


class _Analysis:
    """``AnalysisPrimary`` / ``AnalysisSecondary`` (src/model/analysis.rs:219-311): picture
    planes in [0, 255] -> the latent ``y``. ``op`` is bop or hop (there is no SOP analysis
    transform)."""
    component = 0

    def __init__(self, eng: Engine, params, op: str):
        self.eng = eng
        self.op = op
        self._h = ctypes.c_void_p()
        if isinstance(params, Checkpoint):
            check(lib().zjai_analysis_create_from_checkpoint(eng.handle, _lib.OPS[op], self.component,
                                                             eng.dtype, params.handle,
                                                             ctypes.byref(self._h)), eng.handle)
        else:
            n, c_names, c_ndims, c_dims, c_ptrs, _keep = _descriptors(params)
            check(lib().zjai_analysis_create(eng.handle, _lib.OPS[op], self.component, eng.dtype, n,
                                             c_names, c_ndims, c_dims, c_ptrs, ctypes.byref(self._h)),
                  eng.handle)

    @classmethod
    def load(cls, params, op: str, eng: Engine):
        """``AnalysisPrimary::load(ck, op, eng)``: ``params`` is a ``weights.Checkpoint`` or maps
        checkpoint names to arrays."""
        return cls(eng, params, op)

    def forward(self, eng: Engine, x: np.ndarray, clip: bool = False) -> np.ndarray:
        """``forward`` / ``forward_clip``: planar ``[c, h, w]`` -> ``[chs, h / d, w / d]``."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        c, h, w = x.shape
        d, chs = (16, 160) if self.component == 0 else (8, 96)
        out = np.empty((chs, -(-h // d), -(-w // d)), np.float32)
        check(lib().zjai_analysis_forward(eng.handle, self._h, _fp(x), c, h, w, int(clip), _fp(out),
                                          out.size), eng.handle)
        return out

    def __del__(self):
        try:
            if self._h:
                lib().zjai_net_destroy(self._h)
                self._h = None
        except Exception:
            pass


class AnalysisPrimary(_Analysis):
    component = 0


class AnalysisSecondary(_Analysis):
    component = 1
