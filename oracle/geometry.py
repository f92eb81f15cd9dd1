"""Integer tiling geometry of the synthesis stage, restated in Python. TEST INFRASTRUCTURE ONLY.

Follows ``src/tools/tiles.rs:22-229`` (``synthesis_tiles``, ``region_tiles``, ``latent_extent``),
``src/tools/regions.rs:47-150`` (``axis_coords``, ``grid``, ``region_grid``) and the encoder-side
header choices ``src/encoder/tiles.rs:271-317`` (``conformance_tile_size``, ``synthesis_tiling``)
and ``src/encoder/mod.rs:216-231`` (``region_counts``).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

SYNTHESIS_DOWNSCALE = 16
SYNTHESIS_SAMPLES_PER_TILE = 1 << 20
SYNTHESIS_TILE_OVERLAP = 64
IND_REGION_SYNTHESIS_OVERLAP = 128
NUM_SAMPLES_IN_REGION = 1_048_576


class GeometryError(ValueError):
    pass


@dataclass(frozen=True)
class Area:
    x: int
    y: int
    width: int
    height: int


@dataclass(frozen=True)
class SynthesisTile:
    image: Area
    latent: Area
    core: Area
    core_offset: tuple


@dataclass(frozen=True)
class RegionGrid:
    rows: int
    columns: int
    core: tuple
    extended: tuple


def _ceil(a, b):
    return -(-a // b)


def latent_extent(pos, length, latent_len):
    if length % SYNTHESIS_DOWNSCALE and _ceil(pos + length, SYNTHESIS_DOWNSCALE) < latent_len:
        raise GeometryError("unaligned synthesis tile inside the picture")
    return _ceil(length, SYNTHESIS_DOWNSCALE)


def _contains(r, x, y):
    return r.x <= x < r.x + r.width and r.y <= y < r.y + r.height


def synthesis_tiles(height, width, latent_h, latent_w, tiling=None, regions=None):
    """``tiling`` = ``(tile_size, overlap)`` or None; ``regions`` = RegionGrid or None."""
    if tiling is None:
        image = Area(0, 0, width, height)
        return [SynthesisTile(image, Area(0, 0, latent_w, latent_h), image, (0, 0))]
    size, overlap = tiling
    tile_h, tile_w = min(size, height), min(size, width)
    half = overlap // 2
    if regions is not None:
        return _region_tiles(height, width, latent_h, latent_w, tile_h, tile_w, half, regions)
    if tile_h <= overlap or tile_w <= overlap:
        raise GeometryError("synthesis tile not larger than its overlap")
    tiles = []
    for y in range(0, height - overlap, tile_h - overlap):
        for x in range(0, width - overlap, tile_w - overlap):
            image = Area(x, y, min(tile_w, width - x), min(tile_h, height - y))
            latent = Area(x // SYNTHESIS_DOWNSCALE, y // SYNTHESIS_DOWNSCALE,
                          latent_extent(image.x, image.width, latent_w),
                          latent_extent(image.y, image.height, latent_h))
            if latent.x + latent.width > latent_w or latent.y + latent.height > latent_h:
                raise GeometryError("synthesis tile outside the latent")
            left = 0 if image.x == 0 else half
            top = 0 if image.y == 0 else half
            right = 0 if image.x + image.width >= width else half
            bottom = 0 if image.y + image.height >= height else half
            if image.width <= left + right or image.height <= top + bottom:
                raise GeometryError("synthesis tile is all overlap")
            tiles.append(SynthesisTile(
                image, latent,
                Area(image.x + left, image.y + top, image.width - left - right,
                     image.height - top - bottom), (left, top)))
    return tiles


def _region_tiles(height, width, latent_h, latent_w, tile_h, tile_w, half, regions):
    tiles = []
    for ty in range(0, height, tile_h):
        for tx in range(0, width, tile_w):
            x, y = tx, ty
            w, h = min(tile_w, width - tx), min(tile_h, height - ty)
            x_end, y_end = x + w - 1, y + h - 1
            for r in regions.extended:
                if not (_contains(r, x, y) and _contains(r, x_end, y_end)):
                    continue
                if y > r.y:
                    if y < half:
                        raise GeometryError("tile overlap")
                    y -= half
                    h += half
                if x > r.x:
                    if x < half:
                        raise GeometryError("tile overlap")
                    x -= half
                    w += half
                if y_end < r.y + r.height - 1:
                    h += min(half, max(height - (y + h), 0))
                if x_end < r.x + r.width - 1:
                    w += min(half, max(width - (x + w), 0))
            image = Area(x, y, w, h)
            if x + w > width or y + h > height:
                raise GeometryError("synthesis tile outside the picture")
            latent = Area(x // SYNTHESIS_DOWNSCALE, y // SYNTHESIS_DOWNSCALE,
                          latent_extent(x, w, latent_w), latent_extent(y, h, latent_h))
            if latent.x + latent.width > latent_w or latent.y + latent.height > latent_h:
                raise GeometryError("synthesis tile outside the latent")
            cx, cy, cw, ch = x, y, w, h
            left = top = 0
            bx, by = x + w - 1, y + h - 1
            for r in regions.extended:
                if not (_contains(r, cx, cy) and _contains(r, bx, by)):
                    continue
                if cy > r.y:
                    top += half
                    cy += half
                    if ch < half:
                        raise GeometryError("tile overlap")
                    ch -= half
                if cx > r.x:
                    left += half
                    cx += half
                    if cw < half:
                        raise GeometryError("tile overlap")
                    cw -= half
                ch = min(ch, tile_h)
                cw = min(cw, tile_w)
            if cw == 0 or ch == 0 or left + cw > w or top + ch > h:
                raise GeometryError("synthesis tile is all overlap")
            tiles.append(SynthesisTile(image, latent, Area(cx, cy, cw, ch), (left, top)))
    return tiles


def axis_coords(size, num_regions, depth, partitioned):
    feature = _ceil(size, 1 << depth)
    if not partitioned:
        return [(0, feature)]
    region_size = (_ceil(size, 128) // num_regions) * 128
    out = []
    for i in range(num_regions):
        start = (i * region_size) >> depth
        end = ((i + 1) * region_size) >> depth if i + 1 < num_regions else feature
        out.append((start, end))
    return out


def grid(ver, hor, extend):
    out = []
    for vi, (y0, y1) in enumerate(ver):
        for hi, (x0, x1) in enumerate(hor):
            x, y, width, height = x0, y0, x1 - x0, y1 - y0
            if hi > 0:
                x -= min(extend, x)
                width += extend
            if hi + 1 < len(hor):
                width += extend
            if vi > 0:
                y -= min(extend, y)
                height += extend
            if vi + 1 < len(ver):
                height += extend
            out.append(Area(x, y, width, height))
    return out


def image_region_grid(height, width, rows, columns):
    """``region_grid(hdr, 0, Plane::Image)`` for independent regions (extension 0)."""
    ver = axis_coords(height, rows, 0, True)
    hor = axis_coords(width, columns, 0, True)
    g = tuple(grid(ver, hor, 0))
    return RegionGrid(rows, columns, g, g)


@dataclass(frozen=True)
class Regions:
    """``Regions`` of a picture header: counts, independence, signalled overlaps."""
    num_ver: int
    num_hor: int
    independent: bool = True
    hyper_decoder_overlap: int = 0
    mcm_overlap: int = 0


# ``Plane`` (src/tools/regions.rs:103-114) -> (depth, extension from (hd, mcm) overlaps).
_PLANES = {
    "latent": (4, lambda hd, mcm: mcm >> 1),
    "psi": (5, lambda hd, mcm: mcm >> 2),
    "hyper_latent": (6, lambda hd, mcm: hd),
    "image": (0, lambda hd, mcm: 64 * hd),
}


def region_grid(height, width, ccs, regions, plane):
    """``region_grid(hdr, ccs, plane)`` (src/tools/regions.rs:120-150); ``regions`` None = not
    partitioned. Chroma grids are built on the half-size plane scaled back up by 2."""
    h, w = (height, width) if ccs == 0 else (2 * _ceil(height, 2), 2 * _ceil(width, 2))
    r = regions if regions is not None else Regions(1, 1, False, 0, 0)
    partitioned = regions is not None
    hd, mcm = r.hyper_decoder_overlap * 2, r.mcm_overlap * 4
    depth, ext = _PLANES[plane]
    extend = 0 if r.independent else ext(hd, mcm)
    ver = axis_coords(h, r.num_ver, depth, partitioned)
    hor = axis_coords(w, r.num_hor, depth, partitioned)
    return RegionGrid(r.num_ver, r.num_hor, tuple(grid(ver, hor, 0)), tuple(grid(ver, hor, extend)))


def hyper_crop(length, divider):
    """Rows / columns the hyper-decoder crops (src/decoder/reconstruct.rs:67-69)."""
    return 2 * _ceil(length, 2 * divider) - _ceil(length, divider)


def region_counts(height, width):
    if height * width <= NUM_SAMPLES_IN_REGION:
        return None
    step = int(math.sqrt(NUM_SAMPLES_IN_REGION))
    num_hor = min(max(width // step, 1), _ceil(width, 512))
    num_ver = min(max(height // step, 1), _ceil(height, 256))
    return num_ver, num_hor


def conformance_tile_size(height, width, num_ver, num_hor):
    ver = (_ceil(height, 128) // num_hor) * 128
    hor = (_ceil(width, 128) // num_ver) * 128
    if ver <= height and hor <= width:
        return math.gcd(ver, hor)
    if ver <= height:
        return ver
    if hor <= width:
        return hor
    return 10000


def synthesis_tiling(height, width, independent_regions=None):
    """Header ``(tile_size, overlap)`` or None (``src/encoder/tiles.rs:294-317``)."""
    if independent_regions is not None:
        nv, nh = independent_regions
        size = conformance_tile_size(height, width, nv, nh)
        if size * size >= height * width:
            return None
        return (_ceil(size, 16) * 16, IND_REGION_SYNTHESIS_OVERLAP)
    if SYNTHESIS_SAMPLES_PER_TILE >= height * width:
        return None
    size = int(math.floor(math.sqrt(SYNTHESIS_SAMPLES_PER_TILE)))
    return (_ceil(size, 16) * 16, SYNTHESIS_TILE_OVERLAP)
