"""CPU pins of the latent-reconstruction oracle (hyper-decoder, multi-stage context model,
region geometry and merges; src/model/hyper_decoder.rs, src/model/mcm.rs,
src/decoder/reconstruct.rs:81-234, src/tools/regions.rs) and of the library's host-side region
geometry. The reference holds no vectors for these functions (its tests need trained models), so
the oracle is pinned by closed forms: zero and delta weights make every network an explicit
index map, which a wrong stage position, cat order, transposed-conv orientation, crop, window or
merge offset breaks."""

import itertools

import numpy as np
import pytest

import oracle.graphs as og
from oracle import geometry as geo
from zenjpegai_amd import model, synth


def _ceil(a, b):
    return -(-a // b)


# ------------------------------------------------------------------------------ geometry
def _union_is_partition(areas, h, w):
    cover = np.zeros((h, w), np.int32)
    for a in areas:
        cover[a.y:a.y + a.height, a.x:a.x + a.width] += 1
    return bool((cover == 1).all())


@pytest.mark.parametrize("height,width,ccs", [(2160, 3840, 0), (2160, 3840, 1), (1400, 2096, 0),
                                              (1001, 777, 1), (3000, 2000, 0)])
@pytest.mark.parametrize("rows,cols", [(1, 1), (2, 3), (3, 2)])
def test_region_cores_tile_each_plane_at_its_depth(height, width, ccs, rows, cols):
    """Cores partition the plane at 1/16 (latent), 1/32 (psi), 1/64 (z) and 1 (image); chroma
    grids are built on 2 * ceil(size / 2) (src/tools/regions.rs:120-127)."""
    h, w = (height, width) if ccs == 0 else (2 * _ceil(height, 2), 2 * _ceil(width, 2))
    regions = geo.Regions(rows, cols, independent=True)
    for plane, depth in (("latent", 4), ("psi", 5), ("hyper_latent", 6), ("image", 0)):
        g = geo.region_grid(height, width, ccs, regions, plane)
        assert len(g.core) == rows * cols
        assert _union_is_partition(g.core, _ceil(h, 1 << depth), _ceil(w, 1 << depth))
        assert g.extended == g.core  # independent regions are not extended


def test_region_extension_follows_the_signalled_overlaps():
    """HyperDecoderOverlap = 2 x signalled, McmOverlap = 4 x signalled; the latent plane extends
    by McmOverlap / 2, psi by / 4, z by the hyper overlap, the image by 64 x it -- towards
    neighbours only (src/tools/regions.rs:128-145, :73-101)."""
    r = geo.Regions(2, 3, independent=False, hyper_decoder_overlap=3, mcm_overlap=5)
    hd, mcm = 6, 20
    for plane, ext in (("latent", mcm // 2), ("psi", mcm // 4), ("hyper_latent", hd),
                       ("image", 64 * hd)):
        g = geo.region_grid(2160, 3840, 0, r, plane)
        for i, (c, e) in enumerate(zip(g.core, g.extended)):
            row, col = divmod(i, 3)
            left = min(ext, c.x) if col > 0 else 0
            top = min(ext, c.y) if row > 0 else 0
            assert (e.x, e.y) == (c.x - left, c.y - top)
            assert e.width == c.width + (ext if col > 0 else 0) + (ext if col < 2 else 0)
            assert e.height == c.height + (ext if row > 0 else 0) + (ext if row < 1 else 0)


def test_region_axis_kats_through_the_grid():
    """src/tools/regions.rs:155-170 KATs seen through region_grid: 3000 rows in 3 regions split
    at latent rows 64 and 128 (region size 1024), z rows 16 / 32; one region covers 56 latent
    columns of 888."""
    r = geo.Regions(3, 1)
    g = geo.region_grid(3000, 100, 0, r, "latent")
    assert [(a.y, a.y + a.height) for a in g.core] == [(0, 64), (64, 128), (128, 188)]
    g = geo.region_grid(3000, 100, 0, r, "hyper_latent")
    assert [(a.y, a.y + a.height) for a in g.core] == [(0, 16), (16, 32), (32, 47)]
    g = geo.region_grid(100, 888, 0, None, "latent")
    assert [(a.x, a.width) for a in g.core] == [(0, 56)]


@pytest.mark.parametrize("height,width", [(2160, 3840), (1400, 2096), (999, 1333), (64, 64)])
@pytest.mark.parametrize("ccs", [0, 1])
@pytest.mark.parametrize("regions", [None, geo.Regions(2, 3, True), geo.Regions(2, 2, False, 2, 3),
                                     geo.Regions(3, 1, False, 1, 1)])
def test_library_region_grid_equals_the_oracle(height, width, ccs, regions):
    mr = None if regions is None else model.Regions(regions.num_ver, regions.num_hor,
                                                    regions.independent,
                                                    regions.hyper_decoder_overlap,
                                                    regions.mcm_overlap)
    for plane in ("latent", "psi", "hyper_latent", "image"):
        core, ext = model.region_grid(height, width, ccs, mr, plane)
        want = geo.region_grid(height, width, ccs, regions, plane)
        assert [(a.x, a.y, a.width, a.height) for a in core] == \
            [(a.x, a.y, a.width, a.height) for a in want.core]
        assert [(a.x, a.y, a.width, a.height) for a in ext] == \
            [(a.x, a.y, a.width, a.height) for a in want.extended]


def test_hyper_crop_gives_the_psi_size():
    """2 ceil(z) - hyper_crop = ceil(len / 32) (luma) and ceil(ceil(len / 2) / 16) (chroma) for
    an unpartitioned picture, so the hyper-decoder output is exactly psi."""
    for n in range(1, 3000, 7):
        assert 2 * _ceil(n, 64) - geo.hyper_crop(n, 32) == _ceil(n, 32)
        m = _ceil(n, 2)
        assert 2 * _ceil(2 * m, 64) - geo.hyper_crop(m, 16) == _ceil(m, 16)


# ------------------------------------------------------------------- delta-weight networks
def _delta_params(c, context=True):
    """Weights that turn each network into an index map:
    hyper-decoder: conv1 = I, convT tap (1, 1) = I (input (y, x) -> output (2y, 2x)),
    conv3 = centre-tap I + bias 0.25, conv4 = centre-tap [I; I; I; I] + bias (k + 1) / 8;
    context model: stage 0 fusion picks psi_0; stage s > 0 conv.0 picks stage s - 1 from the
    context, conv.1 is the centre-tap grouped identity, fusion conv1 picks the conv.1 half for
    odd s and the psi half for even s; fusion conv2 = conv3 = I."""
    eye = np.eye(c, dtype=np.float32)
    p = {}
    p["hyper_decoder.conv1.weight"] = eye[:, :, None, None].copy()
    w = np.zeros((c, c, 4, 4), np.float32)
    w[:, :, 1, 1] = eye
    p["hyper_decoder.conv2.weight"] = w
    p["hyper_decoder.conv2.bias"] = np.zeros(c, np.float32)
    w = np.zeros((c, c, 3, 3), np.float32)
    w[:, :, 1, 1] = eye
    p["hyper_decoder.conv3.weight"] = w
    p["hyper_decoder.conv3.bias"] = np.full(c, 0.25, np.float32)
    w = np.zeros((4 * c, c, 3, 3), np.float32)
    for k in range(4):
        w[k * c:(k + 1) * c, :, 1, 1] = eye
    p["hyper_decoder.conv4.weight"] = w
    p["hyper_decoder.conv4.bias"] = np.repeat(np.arange(1, 5, dtype=np.float32) / 8, c)
    if not context:
        return p
    for s in range(4):
        pfx = f"context.MCM.{s}"
        if s > 0:
            w = np.zeros((c, s * c, 1, 1), np.float32)
            w[:, (s - 1) * c:s * c, 0, 0] = eye
            p[f"{pfx}.conv.0.weight"] = w
            w = np.zeros((c, 32, 3, 3), np.float32)
            w[np.arange(c), np.arange(c) % 32, 1, 1] = 1.0
            p[f"{pfx}.conv.1.weight"] = w
            p[f"{pfx}.conv.1.bias"] = np.zeros(c, np.float32)
            w = np.zeros((c, 2 * c, 1, 1), np.float32)
            w[:, (0 if s % 2 else c):(c if s % 2 else 2 * c), 0, 0] = eye
        else:
            w = eye[:, :, None, None].copy()
        p[f"{pfx}.fusion_pred_net.conv1.weight"] = w
        p[f"{pfx}.fusion_pred_net.conv2.weight"] = eye[:, :, None, None].copy()
        p[f"{pfx}.fusion_pred_net.conv3.weight"] = eye[:, :, None, None].copy()
    return p


def _psi_closed_form(z, out_h, out_w):
    """psi of the delta hyper-decoder: quarter k at (2y, 2x) = relu6(relu6(z) + 0.25) + (k+1)/8,
    at odd positions relu6(0 + 0.25) + (k + 1) / 8."""
    c = z.shape[0]
    up = np.zeros((c, 2 * z.shape[1], 2 * z.shape[2]), np.float32)
    up[:, 0::2, 0::2] = z
    up = up[:, :out_h, :out_w]
    inner = np.clip(np.clip(up, 0, 6) + np.float32(0.25), 0, 6)
    return np.concatenate([inner + np.float32((k + 1) / 8) for k in range(4)]).astype(np.float32)


def _y_closed_form(psi, res):
    """y_hat of the delta context model, written per sample: stage s at cell position
    STAGE_POSITIONS[s]; mean_0 = relu(psi_0), mean_s = relu(stage_{s-1}) for odd s, relu(psi_s)
    for even s; a stage sample adds its residual where the latent sample exists."""
    c, h, w = res.shape
    hh, hw = psi.shape[1], psi.shape[2]
    stages = np.zeros((4, c, hh, hw), np.float32)
    y = np.zeros_like(res)
    pos = [(0, 0), (1, 1), (0, 1), (1, 0)]
    for s in range(4):
        for ch, yy, xx in itertools.product(range(c), range(hh), range(hw)):
            if s % 2:
                m = max(stages[s - 1, ch, yy, xx], np.float32(0))
            else:
                m = max(psi[s * c + ch, yy, xx], np.float32(0))
            sy, sx = 2 * yy + pos[s][0], 2 * xx + pos[s][1]
            if sy < h and sx < w:
                m = np.float32(m + res[ch, sy, sx])
                y[ch, sy, sx] = m
            stages[s, ch, yy, xx] = m
    return y


def test_delta_hyper_decoder_is_the_closed_form():
    c = 32
    z = synth.hyper_latent(5, "dz", c, 5, 7, b=3.0)
    p = _delta_params(c)
    for oh, ow in ((10, 14), (9, 13), (7, 8)):
        got = og.hyper_decoder(p, z, oh, ow)
        assert got.shape == (4 * c, oh, ow)
        assert np.array_equal(got, _psi_closed_form(z.astype(np.float32), oh, ow))


@pytest.mark.parametrize("h,w", [(8, 12), (7, 9), (1, 1), (5, 2)])
def test_delta_context_model_is_the_closed_form(h, w):
    c = 32
    p = _delta_params(c)
    res = synth.residual(6, "dr", c, h, w, b=2.0)
    psi = synth.laplace(6, "dpsi", (4 * c, _ceil(h, 2), _ceil(w, 2)), 2.0)
    assert np.array_equal(og.context_decompress(p, res, psi), _y_closed_form(psi, res))


def test_zero_context_model_returns_the_residual():
    c = 32
    p = {k: np.zeros_like(v) for k, v in _delta_params(c).items()}
    res = synth.residual(7, "zr", c, 9, 11)
    psi = synth.laplace(7, "zpsi", (4 * c, 5, 6), 3.0)
    assert np.array_equal(og.context_decompress(p, res, psi), res)


def test_upshuffle_is_the_stage_lut():
    """mean(y, x) = psi[STAGE_LUT[(y % 2) * 2 + x % 2] C + c](y / 2, x / 2), LUT (0, 2, 3, 1):
    the inverse of the stage positions (0,0), (1,1), (0,1), (1,0)."""
    c = 3
    psi = np.arange(4 * c * 3 * 4, dtype=np.float32).reshape(4 * c, 3, 4)
    got = og.upshuffle_psi(psi, 5, 7)
    pos = [(0, 0), (1, 1), (0, 1), (1, 0)]
    for ch, y, x in itertools.product(range(c), range(5), range(7)):
        s = pos.index((y % 2, x % 2))
        assert got[ch, y, x] == psi[s * c + ch, y // 2, x // 2]


@pytest.mark.parametrize("height,width,regions", [
    (256, 384, None),
    (700, 1000, None),
    (1024, 1536, geo.Regions(2, 3, True)),
    (1024, 1536, geo.Regions(2, 2, False, 1, 4)),
    (900, 1300, geo.Regions(2, 2, False, 2, 8)),
])
@pytest.mark.parametrize("ccs", [0, 1])
def test_delta_reconstruction_is_region_independent(height, width, regions, ccs):
    """With index-map weights every region computes the same values where it overlaps
    another, so the merged psi and y_hat equal the closed forms over the whole picture: wrong
    windows, merge offsets or crops break the equality. (Dependent regions need
    mcm_overlap = 4 x hyper_decoder_overlap for this: then a region's z window, extended by
    2 x hd z samples, upsamples onto its psi window, extended by mcm psi samples. The reference
    places each region's psi at its psi window whatever the overlaps are.)"""
    c = 32
    p = _delta_params(c)
    if ccs == 0:
        lh, lw = _ceil(height, 16), _ceil(width, 16)
        zh, zw = _ceil(height, 64), _ceil(width, 64)
    else:
        lh, lw = _ceil(_ceil(height, 2), 8), _ceil(_ceil(width, 2), 8)
        zh, zw = _ceil(2 * _ceil(height, 2), 64), _ceil(2 * _ceil(width, 2), 64)
    z = synth.hyper_latent(8, "rz", c, zh, zw, b=3.0)
    res = synth.residual(8, "rr", c, lh, lw, b=2.0)
    psi, y = og.reconstruct_latent(p, ccs, height, width, regions, z, res)
    want_psi = _psi_closed_form(z.astype(np.float32), _ceil(lh, 2), _ceil(lw, 2))
    assert np.array_equal(psi, want_psi)
    assert np.array_equal(y, _y_closed_form(want_psi, res))


def test_reconstruction_without_context_model_is_upshuffle_plus_residual():
    c = 32
    p = _delta_params(c, context=False)
    z = synth.hyper_latent(9, "nz", c, 4, 6)
    res = synth.residual(9, "nr", c, 16, 24)
    psi, y = og.reconstruct_latent(p, 0, 256, 384, None, z, res, context=False)
    assert np.array_equal(y, og.upshuffle_psi(psi, 16, 24) + res)


def test_latent_parameter_specs_match_the_loaders():
    """Shapes of HyperDecoder::load (hyper_decoder.rs:24-45) and ContextModel::load
    (mcm.rs:123-159): conv.0 s C -> C, conv.1 grouped C / 32, fusion 2C -> C after stage 0."""
    specs = {n: s for n, s, _ in synth.latent_param_specs(1)}
    c = 96
    assert specs["hyper_decoder.conv2.weight"] == (c, c, 4, 4)
    assert specs["hyper_decoder.conv4.weight"] == (4 * c, c, 3, 3)
    assert specs["context.MCM.3.conv.0.weight"] == (c, 3 * c, 1, 1)
    assert specs["context.MCM.2.conv.1.weight"] == (c, 32, 3, 3)
    assert specs["context.MCM.0.fusion_pred_net.conv1.weight"] == (c, c, 1, 1)
    assert specs["context.MCM.1.fusion_pred_net.conv1.weight"] == (c, 2 * c, 1, 1)
    assert "context.MCM.0.conv.0.weight" not in specs
    assert len([n for n in specs if n.startswith("context")]) == 3 + 3 * 6
