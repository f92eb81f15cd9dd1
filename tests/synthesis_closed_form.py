"""Index-map weights for the synthesis nets and the closed forms of their outputs (test helper,
imported by ``test_synthesis_oracle.py`` on the CPU and ``test_gpu_synthesis_closed_form.py``
on the GPU).

With the weights built here every convolution is an index map: each output channel reads ONE
input channel (a fixed affine channel map) at ONE tap (a fixed spatial offset, or one tap per
output phase of a transposed convolution), scaled by a power of two, plus a dyadic bias. Every
convolution output is then a single exact product, whatever order a kernel sums its (zero)
terms in, and each net becomes a composition of shifts, stride-2 samplings, up-samplings,
crops, pixel shuffles and the elementwise gates (relu, relu6, the ResAU gate, the CAB sigmoid
gate, the residual adds). The closed forms below evaluate that composition with numpy index
arithmetic on float32 arrays -- they never call a convolution -- following the layer lists of
``src/model/synthesis.rs`` (LightPrimary :550-580, HopPrimary :356-390, SynthesisSecondary
:1004-1038 with LightSecondary :884-909 / HopSecondary :755-773) and ``src/model/attention.rs``
(ResidualBlock :35-43, Cab :119-139, TransformerBlock :328-372, Tam :528-545).

Families (``Family``):
* ``border=True``: off-centre taps and "ceil" up-sampling (output ``o`` reads input
  ``ceil(o / 2)``, zero past the end), so the zero padding at every map border shows in the
  output: a crop of the wrong size or at the wrong place changes samples near the bottom/right.
  The transformer blocks add position-dependent patterns (layer-norm weight 0, zero queries:
  uniform attention, see ``tab``).
* ``border=False``: centre taps and nearest-neighbour ("floor") up-sampling: every output
  sample depends only on the latent column of its 16 x 16 block, so a tiled picture equals the
  untiled net (``local_picture``); the transformer blocks are identities (zero projections).
* ``gates=False``: residual blocks, ResAU gates and the CAB mask branch reduce to identities /
  constants, so every intermediate value is a small integer or half-integer, exact in f16 and
  bf16 as well (for the 16-bit kernels).

The sigmoid of the CAB gate and the final ``denormalize`` use the oracle's pinned primitives
(``oracle.sigmoid``, the reference's Cephes form; ``oracle.denormalize``).
"""

from __future__ import annotations

import numpy as np

import oracle
from zenjpegai_amd import synth

F32 = np.float32


def _ceil(a, b):
    return -(-a // b)


class Family:
    def __init__(self, border=True, gates=True, out_shift=0):
        self.border, self.gates, self.out_shift = border, gates, out_shift

    def with_shift(self, s):
        return Family(self.border, self.gates, s)

    def __repr__(self):
        return f"Family(border={self.border}, gates={self.gates}, out_shift={self.out_shift})"


# ------------------------------------------------------------------------------ channel maps
def amap(a, b, n):
    """Channel map k -> (a k + b) mod n."""
    return lambda k: (a * k + b) % n


# ------------------------------------------------------------------------- closed-form ops
def read(x, dy, dx):
    """out[c, y, x] = x[c, y + dy, x + dx], zero outside the map."""
    c, h, w = x.shape
    out = np.zeros_like(x)
    y0, y1 = max(0, -dy), min(h, h - dy)
    x0, x1 = max(0, -dx), min(w, w - dx)
    if y0 < y1 and x0 < x1:
        out[:, y0:y1, x0:x1] = x[:, y0 + dy:y1 + dy, x0 + dx:x1 + dx]
    return out


def sample2(x, dy, dx):
    """Stride-2 sampling: out[c, q, r] = x[c, 2q + dy, 2r + dx] (zero outside), ceil(h/2) rows."""
    c, h, w = x.shape
    oh, ow = _ceil(h, 2), _ceil(w, 2)
    pad = np.zeros((c, 2 * oh + 2, 2 * ow + 2), x.dtype)
    pad[:, 1:h + 1, 1:w + 1] = x
    return np.ascontiguousarray(pad[:, 1 + dy:1 + dy + 2 * oh:2, 1 + dx:1 + dx + 2 * ow:2])


def up2(x, ceil):
    """2x up-sampling to 2h x 2w: out[o] = x[ceil(o / 2)] (zero when that is h) or x[o // 2]."""
    c, h, w = x.shape
    oy, ox = np.arange(2 * h), np.arange(2 * w)
    if not ceil:
        return np.ascontiguousarray(x[:, oy // 2][:, :, ox // 2])
    pad = np.zeros((c, h + 1, w + 1), x.dtype)
    pad[:, :h, :w] = x
    return np.ascontiguousarray(pad[:, (oy + 1) // 2][:, :, (ox + 1) // 2])


def shuffle(x, r):
    """Pixel shuffle: out[c, r y + i, r x + j] = x[c r^2 + r i + j, y, x]."""
    c, h, w = x.shape
    return np.ascontiguousarray(
        x.reshape(c // (r * r), r, r, h, w).transpose(0, 3, 1, 4, 2).reshape(c // (r * r), h * r, w * r))


def crop(x, h, w):
    assert h <= x.shape[1] and w <= x.shape[2], (x.shape, h, w)
    return np.ascontiguousarray(x[:, :h, :w])


def chan(x, n, src):
    """n output channels, channel k = x[src(k)]."""
    return np.ascontiguousarray(x[[src(k) for k in range(n)]])


def in_range_sum(h, w, taps):
    """sum over 3x3 taps (ty, tx) of taps[ty][tx] * [the tap's input (y+ty-1, x+tx-1) is inside
    the h x w map], as float64."""
    s = np.zeros((h, w), np.float64)
    ys, xs = np.arange(h)[:, None], np.arange(w)[None, :]
    for ty in range(3):
        for tx in range(3):
            ok = (ys + ty - 1 >= 0) & (ys + ty - 1 < h) & (xs + tx - 1 >= 0) & (xs + tx - 1 < w)
            s += taps[ty][tx] * ok
    return s


# ------------------------------------------------- the layer choices shared by weights and forms
# Spatial offsets (dy, dx) read by the stride-1 3x3 convolutions of the border family; the local
# family reads the centre.
OFF = {"rb1": (1, 1), "rb2": (1, 0), "resau": (-1, 1), "light1": (0, 1), "conv3": (1, -1),
       "combine": (-1, 0)}
OFF_S2 = {"cab": (1, 1), "tam": (1, 1)}  # stride-2 3x3: reads (2q + dy, 2r + dx)
TAP_T1 = [[2.0 ** -(3 * ty + tx) for tx in range(3)] for ty in range(3)]  # attention depthwise
TAP_T2 = [[0.5, 0.0, 0.0], [0.0, 1.0, 0.0], [0.0, 0.0, 0.25]]  # feed-forward depthwise


# Biases: dyadic with gates, integers without (every value then stays a small integer or
# half-integer, exact in bf16).
# Transposed convs carry non-zero biases too, so the samples they produce past the end of their
# input (the "ceil" map reads zero there) are not zero.
BIAS = {"light1": (0.25, 1.0), "fs1": (0.125, 1.0), "conv3": (0.5, 1.0), "combine": (0.25, 1.0),
        "c2t": (0.75, 1.0), "us": (0.25, 1.0)}


def _bias(fam, key):
    return BIAS[key][0 if fam.gates else 1]


def _sub_bias(fam, j):
    """Bias of sub-position j of a 1x1 conv feeding a pixel shuffle."""
    return j / 8 if fam.gates else float(j)


def _off(fam, key):
    return OFF[key] if fam.border else (0, 0)


def _off_s2(fam, key):
    return OFF_S2[key] if fam.border else (0, 0)


def _ln_beta(dim):
    return np.array([((i % 4) + 1) / 4 for i in range(dim)], np.float64)


def _ffn_beta(dim):
    return np.array([((i % 3) + 1) / 2 for i in range(dim)], np.float64)


# ------------------------------------------------------------------------------ weights
def _conv(cout, cin_g, kh, kw, src, tap, scale):
    w = np.zeros((cout, cin_g, kh, kw), np.float32)
    for k in range(cout):
        w[k, src(k), tap[0], tap[1]] = scale
    return w


def _conv3(fam, key, cout, cin, src, scale=1.0):
    dy, dx = _off(fam, key)
    return _conv(cout, cin, 3, 3, src, (dy + 1, dx + 1), scale)


def _convt(cin, cout, k, src, ceil, scale=1.0):
    """Stride-2 transposed conv (pad 1): output o = 2 i - 1 + t; ceil: taps t = 0 (odd o, reads
    i = (o + 1) / 2) and t = 1 (even o, i = o / 2); floor: t = 1 (even) and t = 2 (odd,
    i = (o - 1) / 2)."""
    taps = (0, 1) if ceil else (1, 2)
    w = np.zeros((cin, cout, k, k), np.float32)
    for j in range(cout):
        for ty in taps:
            for tx in taps:
                w[src(j), j, ty, tx] = scale
    return w


def _rb(p, fam, pfx, c):
    p[f"{pfx}.conv1.weight"] = _conv3(fam, "rb1", c, c, amap(1, 1, c))
    p[f"{pfx}.conv1.bias"] = np.zeros(c, np.float32)
    p[f"{pfx}.conv2.weight"] = _conv3(fam, "rb2", c, c, amap(1, 2, c), 0.5 if fam.gates else 0.0)
    p[f"{pfx}.conv2.bias"] = np.zeros(c, np.float32)


def _resau(p, fam, pfx, c, groups):
    cg = c // groups
    p[f"{pfx}.conv.weight"] = _conv3(fam, "resau", c, cg, lambda k: (k % cg + 1) % cg)
    p[f"{pfx}.conv2.weight"] = _conv(c, c, 1, 1, amap(1, 3, c), (0, 0), 0.25 if fam.gates else 0.0)


def _cab(p, fam, pfx, c):
    _rb(p, fam, f"{pfx}.residual_trunk.0", c)
    _rb(p, fam, f"{pfx}.residual_trunk.1", c)
    dy, dx = _off_s2(fam, "cab")
    p[f"{pfx}.subscale.weight"] = _conv(c, c, 3, 3, amap(1, 5, c), (dy + 1, dx + 1), 1.0)
    p[f"{pfx}.subscale.bias"] = np.zeros(c, np.float32)
    _rb(p, fam, f"{pfx}.residual_mask2.0", c)
    _rb(p, fam, f"{pfx}.residual_mask3.0", c)
    p[f"{pfx}.upscale.weight"] = _convt(c, c, 3, amap(1, 0, c), fam.border, 1.0 if fam.gates else 0.0)
    p[f"{pfx}.upscale.bias"] = np.full(c, -0.5 if fam.gates else 0.0, np.float32)


def _tab(p, fam, pfx, d):
    """Border family: layer-norm weight 0 (output = its bias), zero queries (uniform attention
    1/c over each head), value channels = constants spread by the depthwise taps, so the block
    adds position-dependent patterns. Otherwise both projections are zero (identity block)."""
    hidden = 4 * d
    on = fam.border and fam.gates
    p[f"{pfx}.prep_data.norm1.weight"] = np.zeros(d, np.float32)
    p[f"{pfx}.prep_data.norm1.bias"] = _ln_beta(d).astype(np.float32)
    w = np.zeros((3 * d, d, 1, 1), np.float32)
    for j in range(d):
        w[2 * d + j, (3 * j) % d] = 1.0
        w[d + j, j] = 1.0  # keys: anything finite (queries are zero)
    p[f"{pfx}.prep_data.conv1.weight"] = w
    p[f"{pfx}.prep_data.conv2.weight"] = np.tile(np.array(TAP_T1, np.float32), (3 * d, 1, 1, 1))
    p[f"{pfx}.attn.temperature"] = np.ones((4, 1, 1), np.float32)
    p[f"{pfx}.attn.project_out.weight"] = _conv(d, d, 1, 1, amap(1, 1, d), (0, 0), 0.5 if on else 0.0)
    p[f"{pfx}.ffn.norm1.weight"] = np.zeros(d, np.float32)
    p[f"{pfx}.ffn.norm1.bias"] = _ffn_beta(d).astype(np.float32)
    w = np.zeros((2 * hidden, d, 1, 1), np.float32)
    for k in range(hidden):
        w[k, k % d] = 1.0
        w[hidden + k, (k + 1) % d] = 0.5
    p[f"{pfx}.ffn.project_in.weight"] = w
    p[f"{pfx}.ffn.dwconv.weight"] = np.tile(np.array(TAP_T2, np.float32), (2 * hidden, 1, 1, 1))
    p[f"{pfx}.ffn.project_out.weight"] = _conv(d, hidden, 1, 1, amap(4, 1, hidden), (0, 0),
                                               0.25 if on else 0.0)


def _tam(p, fam, pfx, d, ds):
    if ds:
        dy, dx = _off_s2(fam, "tam")
        p[f"{pfx}.ds_conv.weight"] = _conv(d, d, 3, 3, amap(1, 0, d), (dy + 1, dx + 1), 1.0)
        p[f"{pfx}.ds_conv.bias"] = np.zeros(d, np.float32)
        p[f"{pfx}.us_conv.weight"] = _convt(d, d, 3, amap(1, 0, d), fam.border)
        p[f"{pfx}.us_conv.bias"] = np.full(d, _bias(fam, "us"), np.float32)
    _tab(p, fam, f"{pfx}.TABs.0", d)
    _tab(p, fam, f"{pfx}.TABs.1", d)


def _shuffle_1x1(p, fam, pfx, cin, r, bias):
    """1x1 conv cin -> cin r^2 feeding a pixel shuffle: sub-position j of channel c reads input
    channel (c + j cin / r^2) mod cin, plus bias ``_sub_bias(j)``."""
    rr = r * r
    cout = cin * rr
    p[f"{pfx}.weight"] = _conv(cout, cin, 1, 1, lambda k: (k // rr + (k % rr) * (cin // rr)) % cin,
                               (0, 0), 1.0)
    if bias:
        p[f"{pfx}.bias"] = np.array([_sub_bias(fam, k % rr) for k in range(cout)], np.float32)


def _sop_up(p, fam, pfx, cin, cout):
    """SOP upsample: the 2x2 conv over the bottom/right-padded input to 4 cout channels, then
    pixel shuffle 2: channel 4c + j reads input channel (2c + 3j) mod cin at tap
    (1 - j // 2, 1 - j % 2) (border: output o reads x[o // 2 + 1 - o % 2], so the last even row
    reads the row below it) or (0, 0) (local: x[o // 2])."""
    w = np.zeros((4 * cout, cin, 2, 2), np.float32)
    for c in range(cout):
        for j in range(4):
            ty, tx = _sop_tap(fam, j)
            w[4 * c + j, (2 * c + 3 * j) % cin, ty, tx] = 1.0
    p[f"{pfx}.conv.weight"] = w


def _sop_tap(fam, j):
    return (1 - j // 2, 1 - j % 2) if fam.border else (0, 0)


def _sop_up_src(c, j, cin):
    return (2 * c + 3 * j) % cin


def params(op, comp, fam):
    """Index-map parameters of one net (names and shapes of ``synth.param_specs``)."""
    p = {}
    s = 2.0 ** -fam.out_shift
    if op == "hop" and comp == "y":
        c = 128
        _rb(p, fam, "first_stage.0.0", 160)
        p["first_stage.1.weight"] = _convt(160, c, 3, amap(1, 17, 160), fam.border)
        p["first_stage.1.bias"] = np.full(c, _bias(fam, "fs1"), np.float32)
        _resau(p, fam, "first_stage.2", c, 4)
        p["conv2_t.weight"] = _convt(c, c, 3, amap(5, 1, c), fam.border)
        p["conv2_t.bias"] = np.full(c, _bias(fam, "c2t"), np.float32)
        _cab(p, fam, "CAB", c)
        _resau(p, fam, "iact2", c, 4)
        _shuffle_1x1(p, fam, "conv3_t", c, 2, True)
        _tam(p, fam, "TAM", c, True)
        _resau(p, fam, "iact3", c, 4)
        p["conv4_t.weight"] = _convt(c, 1, 3, lambda j: 3, fam.border, s)
        p["conv4_t.bias"] = np.zeros(1, np.float32)
    elif op == "hop":
        c = 64
        p["first_stage.conv1.weight"] = _conv3(fam, "combine", 48, 256, amap(7, 3, 256))
        p["first_stage.conv1.bias"] = np.full(48, _bias(fam, "combine"), np.float32)
        p["conv2_t.weight"] = _convt(144, c, 3, amap(9, 2, 144), fam.border)
        p["conv2_t.bias"] = np.full(c, _bias(fam, "c2t"), np.float32)
        _cab(p, fam, "CAB", c)
        _resau(p, fam, "iact2", c, 4)
        _shuffle_1x1(p, fam, "conv3_t", c, 2, True)
        _tam(p, fam, "TAM", c, False)
        _resau(p, fam, "iact3", c, 4)
        p["conv4_t.weight"] = _convt(c, 8, 3, amap(5, 1, c), fam.border, s)
        p["conv4_t.bias"] = np.zeros(8, np.float32)
    elif comp == "y":
        c1, c2, c3 = (64, 32, 32) if op == "sop" else (64, 64, 96)
        p["first_stage.0.0.conv1.weight"] = _conv3(fam, "light1", 160, 160, amap(1, 1, 160))
        p["first_stage.0.0.conv1.bias"] = np.full(160, _bias(fam, "light1"), np.float32)
        if op == "sop":
            _sop_up(p, fam, "first_stage.1", 160, c1)
        else:
            p["first_stage.1.weight"] = _convt(160, c1, 4, amap(3, 7, 160), fam.border)
            p["first_stage.1.bias"] = np.full(c1, _bias(fam, "fs1"), np.float32)
        _resau(p, fam, "first_stage.2", c1, c1 // 16)
        if op == "sop":
            _sop_up(p, fam, "conv2_t", c1, c2)
        else:
            p["conv2_t.weight"] = _convt(c1, c2, 4, amap(5, 1, c1), fam.border)
            p["conv2_t.bias"] = np.full(c2, _bias(fam, "c2t"), np.float32)
        _resau(p, fam, "iact2", c2, c2 // 16)
        p["conv3.weight"] = _conv3(fam, "conv3", c3, c2, amap(3, 1, c2))
        p["conv3.bias"] = np.full(c3, _bias(fam, "conv3"), np.float32)
        _resau(p, fam, "iact3", c3, c3 // 16)
        p["conv4.weight"] = _conv(16, c3, 1, 1, amap(5, 2, c3), (0, 0), s)
    else:
        c2, c3 = (32, 32) if op == "sop" else (64, 128)
        p["first_stage.conv1.weight"] = _conv3(fam, "combine", 48, 256, amap(7, 3, 256))
        p["first_stage.conv1.bias"] = np.full(48, _bias(fam, "combine"), np.float32)
        if op == "sop":
            _sop_up(p, fam, "conv2_t", 144, c2)
        else:
            p["conv2_t.weight"] = _convt(144, c2, 4, amap(9, 2, 144), fam.border)
            p["conv2_t.bias"] = np.full(c2, _bias(fam, "c2t"), np.float32)
        _resau(p, fam, "iact2", c2, c2 // 16)
        p["conv3.weight"] = _conv3(fam, "conv3", c3, c2, amap(3, 1, c2))
        p["conv3.bias"] = np.full(c3, _bias(fam, "conv3"), np.float32)
        _resau(p, fam, "iact3", c3, c3 // 16)
        p["conv4.weight"] = _conv(128, c3, 1, 1, amap(5, 2, c3), (0, 0), s)
    specs = {n: shape for n, shape, _ in synth.param_specs(op, comp)}
    assert set(specs) == set(p), set(specs) ^ set(p)
    for n, shape in specs.items():
        assert p[n].shape == tuple(shape), (n, p[n].shape, shape)
    return p


# ------------------------------------------------------------------------ closed forms
def relu(x):
    return np.maximum(x, F32(0))


def relu6(x):
    return np.clip(x, F32(0), F32(6))


def rb(fam, x):
    """ResidualBlock: x + 1/2 relu(x at two offsets, channels shifted by 1 then 2)."""
    c = x.shape[0]
    dy1, dx1 = _off(fam, "rb1")
    dy2, dx2 = _off(fam, "rb2")
    t = relu(read(chan(x, c, amap(1, 1, c)), dy1, dx1))
    if not fam.gates:
        return x + F32(0)
    return x + F32(0.5) * read(chan(t, c, amap(1, 2, c)), dy2, dx2)


def resau(fam, x, groups):
    """ResAU: x * (1 + 1/4 relu6(in-group neighbour channel at an offset)), channels of the 1x1
    shifted by 3."""
    c = x.shape[0]
    cg = c // groups
    dy, dx = _off(fam, "resau")
    g = chan(relu6(x), c, lambda k: (k // cg) * cg + (k % cg + 1) % cg)
    g = read(g, dy, dx)
    m = F32(0.25 if fam.gates else 0.0) * chan(g, c, amap(1, 3, c))
    return x * (F32(1) + m)


def cab(fam, x):
    """Cab: x + trunk * sigmoid(mask), trunk = two residual blocks, mask = stride-2 sample ->
    two residual blocks -> 2x up-sampling - 1/2."""
    c = x.shape[0]
    trunk = rb(fam, rb(fam, x))
    m = sample2(chan(x, c, amap(1, 5, c)), *_off_s2(fam, "cab"))
    m = rb(fam, rb(fam, m))
    if fam.gates:
        m = up2(m, fam.border) + F32(-0.5)
    else:
        m = np.zeros_like(x)
    return x + trunk * oracle.sigmoid(m)


def tab(fam, x):
    """TransformerBlock with the weights of ``_tab``: the attention half adds
    1/2 * mean over the head of channel (o + 1) of beta[3j mod d] * S1, the feed-forward half
    1/4 * f[4o + 1], f[k] = elu(a) b = (beta'[k mod d] S2) (beta'[(k + 1) mod d] S2 / 2), with
    S1 / S2 the in-range sums of the depthwise taps (zero padding at the map border)."""
    if not (fam.border and fam.gates):
        return x + F32(0)
    d, h, w = x.shape
    c = d // 4
    beta, beta2 = _ln_beta(d), _ffn_beta(d)
    s1, s2 = in_range_sum(h, w, TAP_T1), in_range_sum(h, w, TAP_T2)
    head_mean = np.array([np.mean([beta[(3 * j) % d] for j in range((i // c) * c, (i // c + 1) * c)])
                          for i in range(d)])
    attn = np.stack([0.5 * head_mean[(o + 1) % d] * s1 for o in range(d)]).astype(F32)
    x = x + attn
    f = np.stack([0.25 * (beta2[(4 * o + 1) % d] * s2) * (0.5 * beta2[(4 * o + 2) % d] * s2)
                  for o in range(d)]).astype(F32)
    return x + f


def tam(fam, x, ds):
    if ds:
        x = sample2(x, *_off_s2(fam, "tam"))
    x = tab(fam, tab(fam, x))
    if ds:
        x = up2(x, fam.border) + F32(_bias(fam, "us"))
    return x


def _light1(fam, y):
    c = y.shape[0]
    t = read(chan(y, c, amap(1, 1, c)), *_off(fam, "light1")) + F32(_bias(fam, "light1"))
    return relu(t) + y


def _conv3_cf(fam, x, cout):
    t = read(chan(x, cout, amap(3, 1, x.shape[0])), *_off(fam, "conv3"))
    return t + F32(_bias(fam, "conv3"))


def _sop_up_cf(fam, x, cout):
    cin = x.shape[0]
    subs = []
    for j in range(4):
        dy, dx = _sop_tap(fam, j)
        subs.append(read(chan(x, cout, lambda c: _sop_up_src(c, j, cin)), dy, dx))
    stacked = np.stack(subs, 1).reshape(4 * cout, *x.shape[1:])
    return shuffle(stacked, 2)


def _shuffle_1x1_cf(fam, x, r):
    cin = x.shape[0]
    rr = r * r
    t = chan(x, cin * rr, lambda k: (k // rr + (k % rr) * (cin // rr)) % cin)
    t = t + np.array([_sub_bias(fam, k % rr) for k in range(cin * rr)], F32)[:, None, None]
    return shuffle(t, r)


def primary(op, fam, y_hat, h, w, denorm=True):
    """Closed form of SynthesisPrimary::forward for ``params(op, "y", fam)``."""
    s = F32(2.0 ** -fam.out_shift)
    if op == "hop":
        x = rb(fam, y_hat)
        x = up2(chan(x, 128, amap(1, 17, 160)), fam.border) + F32(_bias(fam, "fs1"))
        x = resau(fam, x, 4)
        x = crop(x, _ceil(h, 8), _ceil(w, 8))
        x = up2(chan(x, 128, amap(5, 1, 128)), fam.border) + F32(_bias(fam, "c2t"))
        x = cab(fam, x)
        x = crop(x, _ceil(h, 4), _ceil(w, 4))
        x = resau(fam, x, 4)
        x = _shuffle_1x1_cf(fam, x, 2)
        x = tam(fam, x, True)
        x = crop(x, _ceil(h, 2), _ceil(w, 2))
        x = resau(fam, x, 4)
        x = s * up2(chan(x, 1, lambda j: 3), fam.border)
    else:
        c1, c2, c3 = (64, 32, 32) if op == "sop" else (64, 64, 96)
        x = _light1(fam, y_hat)
        if op == "sop":
            x = _sop_up_cf(fam, x, c1)
        else:
            x = up2(chan(x, c1, amap(3, 7, 160)), fam.border) + F32(_bias(fam, "fs1"))
        x = resau(fam, x, c1 // 16)
        x = crop(x, _ceil(h, 8), _ceil(w, 8))
        if op == "sop":
            x = _sop_up_cf(fam, x, c2)
        else:
            x = up2(chan(x, c2, amap(5, 1, c1)), fam.border) + F32(_bias(fam, "c2t"))
        x = crop(x, _ceil(h, 4), _ceil(w, 4))
        x = resau(fam, x, c2 // 16)
        x = _conv3_cf(fam, x, c3)
        x = resau(fam, x, c3 // 16)
        x = shuffle(s * chan(x, 16, amap(5, 2, c3)), 4)
    return oracle.denormalize(x) if denorm else x


def secondary(op, fam, y_luma, y_chroma, h, w, denorm=True):
    """Closed form of SynthesisSecondary::forward_with for ``params(op, "uv", fam)``."""
    s = F32(2.0 ** -fam.out_shift)
    lh, lw = y_chroma.shape[1:]
    cat = np.concatenate([crop(y_luma, lh, lw), y_chroma])
    info = read(chan(cat, 48, amap(7, 3, 256)), *_off(fam, "combine")) + F32(_bias(fam, "combine"))
    x = np.concatenate([info, y_chroma])
    if op == "hop":
        x = up2(chan(x, 64, amap(9, 2, 144)), fam.border) + F32(_bias(fam, "c2t"))
        x = cab(fam, x)
        x = crop(x, _ceil(h, 8), _ceil(w, 8))
        x = resau(fam, x, 4)
        x = _shuffle_1x1_cf(fam, x, 2)
        x = tam(fam, x, False)
        x = crop(x, _ceil(h, 4), _ceil(w, 4))
        x = resau(fam, x, 4)
        x = shuffle(s * up2(chan(x, 8, amap(5, 1, 64)), fam.border), 2)
    else:
        c2, c3 = (32, 32) if op == "sop" else (64, 128)
        if op == "sop":
            x = _sop_up_cf(fam, x, c2)
        else:
            x = up2(chan(x, c2, amap(9, 2, 144)), fam.border) + F32(_bias(fam, "c2t"))
        x = crop(x, _ceil(h, 8), _ceil(w, 8))
        x = resau(fam, x, c2 // 16)
        x = _conv3_cf(fam, x, c3)
        x = resau(fam, x, c3 // 16)
        x = shuffle(s * chan(x, 128, amap(5, 2, c3)), 8)
    return oracle.denormalize(x) if denorm else x


def fit_shift(op, comp, fam, *lat, h, w):
    """The smallest output shift that keeps every closed-form sample of this net inside
    denormalize's unsaturated range (|x| * 128 < 127.5), so the planes show every value."""
    f0 = fam.with_shift(0)
    v = primary(op, f0, *lat, h, w, False) if comp == "y" else secondary(op, f0, *lat, h, w, False)
    m = float(np.max(np.abs(v)))
    s = 0
    while m * 2.0 ** -s * 128 >= 127:
        s += 1
    return fam.with_shift(s)


def local_picture(op, fam_y, fam_uv, y_hat, uv_hat, height, width, sv=1, sh=1, chunk=1024,
                  denorm=True):
    """Planes of the whole picture for the local family: every 16 x 16 output block depends only
    on the latent column at that block, so the blocks are evaluated for ``chunk`` latent columns
    at a time (laid side by side as a 1 x n latent) and scattered to their picture positions.
    Returns (rec_y [height, width], rec_u, rec_v [ceil(h/sv), ceil(w/sh)]) float32."""
    assert not fam_y.border and (fam_uv is None or not fam_uv.border)
    _, lh, lw = y_hat.shape
    n = lh * lw
    yl = y_hat.reshape(160, n)
    ul = uv_hat.reshape(96, n) if uv_hat is not None else None
    full_y = np.zeros((lh, lw, 16, 16), np.float32)
    full_uv = np.zeros((2, lh, lw, 16, 16), np.float32)
    for a in range(0, n, chunk):
        b = min(n, a + chunk)
        k = b - a
        ty = primary(op, fam_y, yl[:, None, a:b].copy(), 16, 16 * k, denorm)
        blocks = ty[0].reshape(16, k, 16).transpose(1, 0, 2)
        full_y.reshape(n, 16, 16)[a:b] = blocks
        if ul is not None:
            tu = secondary(op, fam_uv, yl[:, None, a:b].copy(), ul[:, None, a:b].copy(), 16,
                           16 * k, denorm)
            full_uv.reshape(2, n, 16, 16)[:, a:b] = tu.reshape(2, 16, k, 16).transpose(0, 2, 1, 3)
    rec_y = full_y.transpose(0, 2, 1, 3).reshape(16 * lh, 16 * lw)[:height, :width]
    rec_uv = full_uv.transpose(0, 1, 3, 2, 4).reshape(2, 16 * lh, 16 * lw)[:, :height:sv, :width:sh]
    return np.ascontiguousarray(rec_y), np.ascontiguousarray(rec_uv[0]), np.ascontiguousarray(rec_uv[1])
