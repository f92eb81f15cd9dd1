"""Graph-level oracle: the synthesis transforms as compositions of the oracle layer loops.
TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Each function restates one forward of the reference's ``src/model/synthesis.rs`` /
``src/model/attention.rs`` op by op; ``p`` maps checkpoint names to numpy arrays (the layouts of
``fuzz/fuzz_targets/common.rs:152-345``). Planar ``[c, h, w]`` float32 throughout.
"""

from __future__ import annotations

import math

import numpy as np

from . import (add, channel_attention, denormalize, elu_gate, gate,
               layer_norm_channels, mul, pixel_shuffle, quantize_plane, relu, relu6, sigmoid)
from . import conv2d as _conv2d
from . import conv_transpose2d as _conv_transpose2d

# Which convolution engine the graphs run on: the nn::reference loops (default) or the restated
# nn::fast blocked engine (the CPU baseline). Both give the same result bit for bit.
_FAST = False


class fast_convs:
    """``with fast_convs(): ...`` runs the graphs' convolutions on the nn::fast restatement."""

    def __enter__(self):
        global _FAST
        self._prev, _FAST = _FAST, True

    def __exit__(self, *exc):
        global _FAST
        _FAST = self._prev


def conv2d(*args, **kw):
    return _conv2d(*args, fast=_FAST, **kw)


def conv_transpose2d(*args, **kw):
    return _conv_transpose2d(*args, fast=_FAST, **kw)


def _ceil(a, b):
    return -(-a // b)


def crop(x, h, w):
    """``BTensor::crop_par``: top-left ``h x w`` corner (src/nn/fast/tensor.rs:349-367)."""
    if h > x.shape[1] or w > x.shape[2]:
        raise ValueError("crop larger than tensor")
    return np.ascontiguousarray(x[:, :h, :w])


def conv3x3(p, name, x, groups=1, stride=1):
    """``load::conv3x3`` layer (src/model/load.rs:46): pad 1."""
    return conv2d(x, p[f"{name}.weight"], p.get(f"{name}.bias"), stride, (1, 1), groups)


def conv1x1(p, name, x):
    return conv2d(x, p[f"{name}.weight"], p.get(f"{name}.bias"), 1, (0, 0), 1)


def conv3x3_t(p, name, x):
    """``attention::conv3x3_t`` (src/model/attention.rs:78-91): k3 s2 p1 op1."""
    return conv_transpose2d(x, p[f"{name}.weight"], p[f"{name}.bias"], 2, 1, 1)


def res_au(p, pfx, x):
    """``ResAu::forward`` (src/model/synthesis.rs:62-74): x * (1 + conv2(conv(relu6(x))))."""
    w = p[f"{pfx}.conv.weight"]
    groups = x.shape[0] // w.shape[1]
    t = conv2d(relu6(x), w, None, 1, (1, 1), groups)
    m = conv1x1(p, f"{pfx}.conv2", t)
    return gate(x, m)


def upsample(p, op, pfx, x):
    """``Upsample::forward`` (src/model/synthesis.rs:117-171)."""
    if op == "bop":
        return conv_transpose2d(x, p[f"{pfx}.weight"], p[f"{pfx}.bias"], 2, 1, 0)
    t = conv2d(x, p[f"{pfx}.conv.weight"], None, 1, (0, 0), 1, extra_pad=(0, 0, 1, 1))
    return pixel_shuffle(t, 2)


def residual_block(p, pfx, x):
    """``ResidualBlock::forward`` (src/model/attention.rs:35-43)."""
    t = relu(conv3x3(p, f"{pfx}.conv1", x))
    return add(conv3x3(p, f"{pfx}.conv2", t), x)


def cab(p, pfx, x):
    """``Cab::forward`` (src/model/attention.rs:119-139): x + trunk(x) * sigmoid(mask(x))."""
    trunk = residual_block(p, f"{pfx}.residual_trunk.0", x)
    trunk = residual_block(p, f"{pfx}.residual_trunk.1", trunk)
    m = conv3x3(p, f"{pfx}.subscale", x, stride=2)
    m = residual_block(p, f"{pfx}.residual_mask2.0", m)
    m = residual_block(p, f"{pfx}.residual_mask3.0", m)
    m = conv3x3_t(p, f"{pfx}.upscale", m)
    if m.shape != trunk.shape:
        raise ValueError("CAB: odd feature map size")
    return add(mul(trunk, sigmoid(m)), x)


def transformer_block(p, pfx, x):
    """``TransformerBlock::forward`` (src/model/attention.rs:328-372), heads 4, hidden 4d."""
    dim = x.shape[0]
    hidden = 4 * dim
    t = layer_norm_channels(x, p[f"{pfx}.prep_data.norm1.weight"], p[f"{pfx}.prep_data.norm1.bias"])
    t = conv1x1(p, f"{pfx}.prep_data.conv1", t)
    t = conv2d(t, p[f"{pfx}.prep_data.conv2.weight"], None, 1, (1, 1), t.shape[0])
    a = channel_attention(t, 4, p[f"{pfx}.attn.temperature"].ravel())
    a = conv1x1(p, f"{pfx}.attn.project_out", a)
    x = add(x, a)
    t = layer_norm_channels(x, p[f"{pfx}.ffn.norm1.weight"], p[f"{pfx}.ffn.norm1.bias"])
    t = conv1x1(p, f"{pfx}.ffn.project_in", t)
    t = conv2d(t, p[f"{pfx}.ffn.dwconv.weight"], None, 1, (1, 1), t.shape[0])
    f = elu_gate(t[:hidden], t[hidden:])
    f = conv1x1(p, f"{pfx}.ffn.project_out", f)
    return add(x, f)


def tam(p, pfx, x, downsample):
    """``Tam::forward`` (src/model/attention.rs:528-545)."""
    if downsample:
        x = conv3x3(p, f"{pfx}.ds_conv", x, stride=2)
    x = transformer_block(p, f"{pfx}.TABs.0", x)
    x = transformer_block(p, f"{pfx}.TABs.1", x)
    if downsample:
        x = conv3x3_t(p, f"{pfx}.us_conv", x)
    return x


def light_primary(p, op, y_hat, h, w, denorm=True):
    """``LightPrimary::forward`` (src/model/synthesis.rs:550-580) -> ``[1, >=h, >=w]``.
    ``denorm=False`` returns the values before ``denormalize`` (for conditioning bounds)."""
    x = add(relu(conv3x3(p, "first_stage.0.0.conv1", y_hat)), y_hat)
    x = upsample(p, op, "first_stage.1", x)
    x = res_au(p, "first_stage.2", x)
    x = crop(x, _ceil(h, 8), _ceil(w, 8))
    x = upsample(p, op, "conv2_t", x)
    x = crop(x, _ceil(h, 4), _ceil(w, 4))
    x = res_au(p, "iact2", x)
    x = conv3x3(p, "conv3", x)
    x = res_au(p, "iact3", x)
    x = pixel_shuffle(conv1x1(p, "conv4", x), 4)
    return denormalize(x) if denorm else x


def hop_primary(p, y_hat, h, w, denorm=True):
    """``HopPrimary::forward`` (src/model/synthesis.rs:356-390)."""
    x = residual_block(p, "first_stage.0.0", y_hat)
    x = conv3x3_t(p, "first_stage.1", x)
    x = res_au(p, "first_stage.2", x)
    x = crop(x, _ceil(h, 8), _ceil(w, 8))
    x = conv3x3_t(p, "conv2_t", x)
    x = cab(p, "CAB", x)
    x = crop(x, _ceil(h, 4), _ceil(w, 4))
    x = res_au(p, "iact2", x)
    x = conv1x1(p, "conv3_t", x)
    x = pixel_shuffle(x, 2)
    x = tam(p, "TAM", x, True)
    x = crop(x, _ceil(h, 2), _ceil(w, 2))
    x = res_au(p, "iact3", x)
    x = conv3x3_t(p, "conv4_t", x)
    return denormalize(x) if denorm else x


def primary(p, op, y_hat, h, w, denorm=True):
    """``SynthesisPrimary::forward`` (src/model/synthesis.rs:262-276)."""
    if op == "hop":
        return hop_primary(p, y_hat, h, w, denorm)
    return light_primary(p, op, y_hat, h, w, denorm)


def secondary(p, op, y_hat_luma, y_hat_chroma, h, w, denorm=True):
    """``SynthesisSecondary::forward_with`` (src/model/synthesis.rs:1004-1038) with
    ``LightSecondary``/``HopSecondary`` tails (:884-909, :755-773)."""
    lh = min(y_hat_luma.shape[1], y_hat_chroma.shape[1])
    lw = min(y_hat_luma.shape[2], y_hat_chroma.shape[2])
    if y_hat_chroma.shape[1:] != (lh, lw):
        raise ValueError("chroma latent larger than the luma latent")
    x = np.concatenate([crop(y_hat_luma, lh, lw), y_hat_chroma], 0)
    info = conv3x3(p, "first_stage.conv1", x)
    x = np.concatenate([info, y_hat_chroma], 0)
    if op == "hop":
        x = conv3x3_t(p, "conv2_t", x)
        x = cab(p, "CAB", x)
        x = crop(x, _ceil(h, 8), _ceil(w, 8))
        x = res_au(p, "iact2", x)
        x = conv1x1(p, "conv3_t", x)
        x = pixel_shuffle(x, 2)
        x = tam(p, "TAM", x, False)
        x = crop(x, _ceil(h, 4), _ceil(w, 4))
        x = res_au(p, "iact3", x)
        x = conv3x3_t(p, "conv4_t", x)
        x = pixel_shuffle(x, 2)
    else:
        x = upsample(p, op, "conv2_t", x)
        x = crop(x, _ceil(h, 8), _ceil(w, 8))
        x = res_au(p, "iact2", x)
        x = conv3x3(p, "conv3", x)
        x = res_au(p, "iact3", x)
        x = conv1x1(p, "conv4", x)
        x = pixel_shuffle(x, 8)
    return denormalize(x) if denorm else x


def synthesize(py, puv, op, y_hat, uv_hat, height, width, tiles, sv=1, sh=1, out_h=None,
               out_w=None, denorm=True):
    """``synthesize_luma_into`` + ``synthesize_chroma_into`` (src/decoder/reconstruct.rs:379-464):
    per tile, window the latents, run the nets, copy tile cores into the planes (chroma keeps the
    rows/cols at multiples of ``sv``/``sh``). ``tiles`` are ``geometry.SynthesisTile``.
    Returns ``(rec_y [out_h, out_w], rec_u, rec_v [ceil(out_h/sv), ceil(out_w/sw)])`` float32;
    ``puv`` None skips chroma. ``denorm=False`` keeps the nets' values before ``denormalize``
    (which is elementwise, so ``denormalize`` of these planes gives the default result)."""
    out_h = height if out_h is None else out_h
    out_w = width if out_w is None else out_w
    rec_y = np.zeros((out_h, out_w), np.float32)
    ch, cw = _ceil(out_h, sv), _ceil(out_w, sh)
    rec_u = np.zeros((ch, cw), np.float32)
    rec_v = np.zeros((ch, cw), np.float32)
    for t in tiles:
        img, lat, core = t.image, t.latent, t.core
        ox, oy = t.core_offset
        by = np.ascontiguousarray(y_hat[:, lat.y:lat.y + lat.height, lat.x:lat.x + lat.width])
        ty = primary(py, op, by, img.height, img.width, denorm)[0]
        rows = min(core.height, max(out_h - core.y, 0))
        cols = min(core.width, max(out_w - core.x, 0))
        rec_y[core.y:core.y + rows, core.x:core.x + cols] = ty[oy:oy + rows, ox:ox + cols]
        if puv is None:
            continue
        buv = np.ascontiguousarray(uv_hat[:, lat.y:lat.y + lat.height, lat.x:lat.x + lat.width])
        tuv = secondary(puv, op, by, buv, img.height, img.width, denorm)
        for c, dst in enumerate((rec_u, rec_v)):
            y0 = _ceil(core.y, sv) * sv
            x0 = _ceil(core.x, sh) * sh
            for py_ in range(y0, min(core.y + core.height, out_h), sv):
                xs = np.arange(x0, min(core.x + core.width, out_w), sh)
                dst[py_ // sv, xs // sh] = tuv[c, oy + py_ - core.y, ox + xs - core.x]
    return rec_y, rec_u, rec_v


__all__ = ["crop", "res_au", "upsample", "residual_block", "cab", "transformer_block", "tam",
           "light_primary", "hop_primary", "primary", "secondary", "synthesize", "quantize_plane",
           "math"]


# ---------------------------------------------------------------------------------------------
# Latent reconstruction: src/model/hyper_decoder.rs, src/model/mcm.rs, src/decoder/reconstruct.rs
# ---------------------------------------------------------------------------------------------

# STAGE_POSITIONS (src/model/mcm.rs:26): (row, column) of stage s inside each 2x2 cell.
STAGE_POSITIONS = ((0, 0), (1, 1), (0, 1), (1, 0))


def hyper_decoder(p, z_hat, out_h, out_w):
    """``HyperDecoder::forward_with`` (src/model/hyper_decoder.rs:58-89): int8 ``[C, hz, wz]``
    -> psi ``[4C, out_h, out_w]``: conv1x1 -> convT4 s2 p1 -> crop -> relu6 -> conv3x3 ->
    relu6 -> conv3x3 (C -> 4C)."""
    x = np.ascontiguousarray(z_hat, dtype=np.float32)
    x = conv1x1(p, "hyper_decoder.conv1", x)
    x = conv_transpose2d(x, p["hyper_decoder.conv2.weight"], p["hyper_decoder.conv2.bias"], 2, 1, 0)
    if x.shape[1:] != (out_h, out_w):
        x = crop(x, out_h, out_w)
    x = relu6(x)
    x = conv3x3(p, "hyper_decoder.conv3", x)
    x = relu6(x)
    return conv3x3(p, "hyper_decoder.conv4", x)


def _fusion(p, pfx, x):
    """``FusionPredNet::forward`` (src/model/mcm.rs:60-66)."""
    x = relu(conv1x1(p, f"{pfx}.conv1", x))
    x = relu(conv1x1(p, f"{pfx}.conv2", x))
    return conv1x1(p, f"{pfx}.conv3", x)


def context_decompress(p, residual, psi):
    """``ContextModel::decompress_with`` (src/model/mcm.rs:171-240): residual ``[C, H, W]``,
    psi ``[4C, ceil(H/2), ceil(W/2)]`` -> y_hat ``[C, H, W]``. Stage s predicts a mean on the
    half-resolution grid from psi quarter s and (s > 0) the stages so far; the stage becomes
    mean + residual where its latent sample exists (padded border samples keep the mean)."""
    c, h, w = residual.shape
    hh, hw = _ceil(h, 2), _ceil(w, 2)
    if psi.shape != (4 * c, hh, hw):
        raise ValueError("context model: residual / psi shape mismatch")
    y_hat = np.zeros((c, h, w), np.float32)
    context = None
    for s, (py, px) in enumerate(STAGE_POSITIONS):
        pfx = f"context.MCM.{s}"
        psi_s = psi[s * c:(s + 1) * c]
        if s == 0:
            mean = _fusion(p, f"{pfx}.fusion_pred_net", psi_s)
        else:
            t = conv1x1(p, f"{pfx}.conv.0", context)
            t = conv3x3(p, f"{pfx}.conv.1", t, groups=c // 32)
            mean = _fusion(p, f"{pfx}.fusion_pred_net", np.concatenate([t, psi_s]))
        stage = mean.copy()
        ys, xs = np.arange(hh) * 2 + py, np.arange(hw) * 2 + px
        iy, ix = np.nonzero(ys < h)[0], np.nonzero(xs < w)[0]
        sub = residual[:, ys[iy]][:, :, xs[ix]]
        stage[:, iy[:, None], ix[None, :]] = (mean[:, iy[:, None], ix[None, :]] + sub).astype(np.float32)
        y_hat[:, ys[iy][:, None], xs[ix][None, :]] = stage[:, iy[:, None], ix[None, :]]
        context = stage if context is None else np.concatenate([context, stage])
    return y_hat


def upshuffle_psi(psi, h, w):
    """``upshuffle_psi_par`` (src/model/mcm.rs:742-764): psi quarters to latent resolution,
    sample (y, x) from quarter STAGE_LUT[(y % 2) * 2 + x % 2] at (y / 2, x / 2)."""
    lut = (0, 2, 3, 1)
    c = psi.shape[0] // 4
    if psi.shape[0] % 4 or psi.shape[1] * 2 < h or psi.shape[2] * 2 < w:
        raise ValueError("upshuffle_psi: shape mismatch")
    out = np.empty((c, h, w), np.float32)
    for py in range(2):
        for px in range(2):
            q = lut[py * 2 + px]
            blk = psi[q * c:(q + 1) * c, :_ceil(h - py, 2), :_ceil(w - px, 2)]
            out[:, py::2, px::2] = blk
    return out


def _assign(dst, core, src, offset):
    """``assign_par`` (src/decoder/reconstruct.rs:38-62): clamped rectangle copy."""
    ox, oy = offset
    h = max(0, min(core.height, src.shape[1] - oy, dst.shape[1] - core.y))
    w = max(0, min(core.width, src.shape[2] - ox, dst.shape[2] - core.x))
    c = min(dst.shape[0], src.shape[0])
    dst[:c, core.y:core.y + h, core.x:core.x + w] = src[:c, oy:oy + h, ox:ox + w]


def _window(t, a):
    if a.y + a.height > t.shape[1] or a.x + a.width > t.shape[2]:
        raise ValueError("window outside tensor")
    return np.ascontiguousarray(t[:, a.y:a.y + a.height, a.x:a.x + a.width])


def reconstruct_latent(p, ccs, height, width, regions, z_hat, residual, context=True):
    """``reconstruct_latent_timed`` (src/decoder/reconstruct.rs:104-234) for component ``ccs``
    of a ``height x width`` picture: ``(psi, y_hat)``. ``context`` says whether the model has
    a context model (else y_hat = up-shuffled psi + residual)."""
    from .geometry import hyper_crop, region_grid
    c, h, w = residual.shape
    img = region_grid(height, width, ccs, regions, "image")
    zg = region_grid(height, width, ccs, regions, "hyper_latent")
    pg = region_grid(height, width, ccs, regions, "psi")
    lg = region_grid(height, width, ccs, regions, "latent")
    psi = np.zeros((4 * c, _ceil(h, 2), _ceil(w, 2)), np.float32)
    for it, zt, core in zip(img.extended, zg.extended, pg.extended):
        th, tw, div = (it.height, it.width, 32) if ccs == 0 else (_ceil(it.height, 2), _ceil(it.width, 2), 16)
        out_h, out_w = 2 * zt.height - hyper_crop(th, div), 2 * zt.width - hyper_crop(tw, div)
        t = hyper_decoder(p, _window(z_hat, zt), out_h, out_w)
        _assign(psi, core, t, (0, 0))
    y_hat = np.zeros((c, h, w), np.float32)
    independent = regions is not None and regions.independent
    for it, lt, pt in zip(img.extended, lg.extended, pg.extended):
        res, ps = _window(residual, lt), _window(psi, pt)
        if context:
            y = context_decompress(p, res, ps)
        else:
            y = (upshuffle_psi(ps, lt.height, lt.width) + res).astype(np.float32)
        if not independent:
            # Picture-border branch of ``_get_core_of_overlapping_tile``: one latent sample
            # (HD_MCM_TILE_OVERLAP / 2 / 16) dropped on every interior side.
            cut = 48 // 2 // 16
            left = 0 if it.x == 0 else cut
            top = 0 if it.y == 0 else cut
            right = 0 if it.x + it.width >= width else cut
            bottom = 0 if it.y + it.height >= height else cut
            core = type(lt)(lt.x + left, lt.y + top, lt.width - left - right, lt.height - top - bottom)
            _assign(y_hat, core, y, (left, top))
        else:
            _assign(y_hat, lt, y, (0, 0))
    return psi, y_hat


# ------------------------------------------------------------------------------ analysis
# The encoder's analysis transforms (src/model/analysis.rs), composed of the pinned layers.

def normalize(x):
    """``normalize`` (src/model/analysis.rs:35-39): (x - 127.5) / 128 in f32."""
    return ((x.astype(np.float32) - np.float32(127.5)) / np.float32(128.0)).astype(np.float32)


def pad_amount(length, divider):
    """``pad_amount`` (src/model/analysis.rs:43-46)."""
    return 2 * _ceil(length, 2 * divider) - _ceil(length, divider)


def replicate_pad(x, bottom, right):
    """``replicate_pad`` (src/model/analysis.rs:48-70): F.pad(x, (0, right, 0, bottom),
    mode="replicate")."""
    if bottom == 0 and right == 0:
        return x
    return np.pad(x, ((0, 0), (0, bottom), (0, right)), mode="edge")


def pad_for(x, h, w, divider):
    """``pad_for`` (src/model/analysis.rs:72-81)."""
    if x.shape[1:] != (_ceil(h, divider), _ceil(w, divider)):
        raise ValueError("analysis transform: map size does not match the picture size")
    return replicate_pad(x, pad_amount(h, divider), pad_amount(w, divider))


def clip_channels(x, lo, hi):
    """``clip_channels`` (src/model/load.rs:103-119): channel c < min(len(lo), len(hi)) clamped
    to [lo[c], hi[c]]; NaN stays NaN."""
    x = x.copy()
    for c in range(min(len(lo), len(hi), x.shape[0])):
        lo_c, hi_c = np.float32(lo[c]), np.float32(hi[c])
        v = x[c]
        v = np.where(v < lo_c, lo_c, v)
        x[c] = np.where(v > hi_c, hi_c, v)
    return x


def _clip(p, op, stage, x, clip):
    key = f"clip_thres.E{stage}{'H' if op == 'hop' else 'B'}"
    if not clip or f"{key}.MinList" not in p or f"{key}.MaxList" not in p:
        return x
    return clip_channels(x, np.asarray(p[f"{key}.MinList"], np.float32).ravel(),
                         np.asarray(p[f"{key}.MaxList"], np.float32).ravel())


def _analysis_trunk(p, op, x, luma, clip):
    """``Trunk::forward`` (src/model/analysis.rs:157-207)."""
    _, h, w = x.shape
    t = conv3x3(p, "conv1", pad_for(normalize(x), h, w, 1), stride=2)
    t = res_au(p, "act1", _clip(p, op, 1, t, clip))
    t = pad_for(t, h, w, 2)
    if op == "hop":
        t = tam(p, "TAM", t, luma)
    t = res_au(p, "act2", _clip(p, op, 2, conv3x3(p, "conv2", t, stride=2), clip))
    t = pad_for(t, h, w, 4)
    if op == "hop":
        t = cab(p, "cab", t)
    return res_au(p, "act3", _clip(p, op, 3, conv3x3(p, "conv3", t, stride=2), clip))


def analysis_primary(p, op, x, clip=False):
    """``AnalysisPrimary::forward_clip`` (src/model/analysis.rs:248-270): [1, h, w] in [0, 255]
    -> [160, ceil(h/16), ceil(w/16)]."""
    if op not in ("bop", "hop"):
        raise ValueError("there is no SOP analysis transform (use BOP)")
    _, h, w = x.shape
    t = pad_for(_analysis_trunk(p, op, x, True, clip), h, w, 8)
    t = _clip(p, op, 4, conv3x3(p, "conv4", t, stride=2), clip)
    return _clip(p, op, 5, conv1x1(p, "conv5", t), clip)


def analysis_secondary(p, op, x, clip=False):
    """``AnalysisSecondary::forward_clip`` (src/model/analysis.rs:297-310): [12, h, w] ->
    [96, ceil(h/8), ceil(w/8)]."""
    if op not in ("bop", "hop"):
        raise ValueError("there is no SOP analysis transform (use BOP)")
    t = _analysis_trunk(p, op, x, False, clip)
    return _clip(p, op, 5, conv1x1(p, "conv5", t), clip)
