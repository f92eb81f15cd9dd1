"""Synthetic workloads: seeded random-init weights of the synthesis nets and random latents.

The reference ships no checkpoints for this path and has no initialiser, so the workloads are
generated:

* PRNG: SplitMix64 over a counter, one stream per tensor (seed mixed with a hash of the tensor's
  name). ``u = (z >> 40) * 2^-24`` gives a uniform in [0, 1) with 24 exact bits.
* Normal: Box-Muller. He-normal std = sqrt(2 / fan_in), fan_in = (in_ch / groups) * kh * kw for a
  convolution and in_ch * (k / stride)^2 for a stride-2 transposed convolution (the mean number
  of taps that reach one output: 4 for k4, 2.25 for k3). Biases N(0, 0.01).
* Layer norm weight 1, bias 0; attention temperature 1 (as the reference's synthetic fuzz models
  set them, ``fuzz/fuzz_targets/common.rs:194-207``).
* Latents: round(Laplace(0, b)), Laplace drawn as ``-b * sgn(u) * ln(1 - 2|u|)``.

Parameter names and shapes are the checkpoint's (``fuzz/fuzz_targets/common.rs:152-345``).
"""

from __future__ import annotations

import hashlib

import numpy as np

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def _splitmix(seed: int, n: int) -> np.ndarray:
    with np.errstate(over="ignore"):
        i = np.arange(1, n + 1, dtype=np.uint64)
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + i * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    return z


def _stream_seed(seed: int, name: str) -> int:
    h = hashlib.sha256(name.encode()).digest()
    return (seed * 0x9E3779B97F4A7C15 + int.from_bytes(h[:8], "little")) & 0xFFFFFFFFFFFFFFFF


def uniform(seed: int, name: str, shape, lo=0.0, hi=1.0) -> np.ndarray:
    n = int(np.prod(shape))
    u = (_splitmix(_stream_seed(seed, name), n) >> np.uint64(40)).astype(np.float64) * 2.0**-24
    return (lo + (hi - lo) * u).astype(np.float32).reshape(shape)


def normal(seed: int, name: str, shape, std=1.0) -> np.ndarray:
    n = int(np.prod(shape))
    z = _splitmix(_stream_seed(seed, name), 2 * n)
    u1 = ((z[0::2] >> np.uint64(40)).astype(np.float64) + 1.0) * 2.0**-24  # (0, 1]
    u2 = (z[1::2] >> np.uint64(40)).astype(np.float64) * 2.0**-24
    g = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    return (g * std).astype(np.float32).reshape(shape)


def laplace(seed: int, name: str, shape, b=1.0) -> np.ndarray:
    n = int(np.prod(shape))
    z = _splitmix(_stream_seed(seed, name), n)
    u = (z >> np.uint64(40)).astype(np.float64) * 2.0**-24 - 0.5  # [-0.5, 0.5)
    u = np.clip(u, -0.5 + 2.0**-25, 0.5 - 2.0**-25)
    x = -b * np.sign(u) * np.log(1.0 - 2.0 * np.abs(u))
    return x.astype(np.float32).reshape(shape)


def latent(seed: int, name: str, c: int, h: int, w: int, b: float = 1.5) -> np.ndarray:
    """``round(Laplace(0, b))`` latent ``[c, h, w]`` (round half away from zero, like Rust's
    ``f32::round``)."""
    x = laplace(seed, name, (c, h, w), b).astype(np.float64)
    return (np.sign(x) * np.floor(np.abs(x) + 0.5)).astype(np.float32)


# ---------------------------------------------------------------------------------------------
# Parameter lists of the synthesis nets (checkpoint names / shapes).
# ---------------------------------------------------------------------------------------------

def _conv3(out, pfx, i, o, bias=True):
    out.append((f"{pfx}.weight", (o, i, 3, 3), "conv"))
    if bias:
        out.append((f"{pfx}.bias", (o,), "bias"))


def _conv1(out, pfx, i, o, bias):
    out.append((f"{pfx}.weight", (o, i, 1, 1), "conv"))
    if bias:
        out.append((f"{pfx}.bias", (o,), "bias"))


def _conv_t(out, pfx, i, o, k):
    out.append((f"{pfx}.weight", (i, o, k, k), "convt"))
    out.append((f"{pfx}.bias", (o,), "bias"))


def _res_au(out, pfx, c, groups):
    out.append((f"{pfx}.conv.weight", (c, c // groups, 3, 3), "conv"))
    out.append((f"{pfx}.conv2.weight", (c, c, 1, 1), "conv"))


def _res_block(out, pfx, c):
    _conv3(out, f"{pfx}.conv1", c, c)
    _conv3(out, f"{pfx}.conv2", c, c)


def _layer_norm(out, pfx, dim):
    out.append((f"{pfx}.weight", (dim,), "ones"))
    out.append((f"{pfx}.bias", (dim,), "zeros"))


def _transformer_block(out, pfx, dim):
    hidden = dim * 4
    _layer_norm(out, f"{pfx}.prep_data.norm1", dim)
    _conv1(out, f"{pfx}.prep_data.conv1", dim, 3 * dim, False)
    out.append((f"{pfx}.prep_data.conv2.weight", (3 * dim, 1, 3, 3), "conv"))
    out.append((f"{pfx}.attn.temperature", (4, 1, 1), "ones"))
    _conv1(out, f"{pfx}.attn.project_out", dim, dim, False)
    _layer_norm(out, f"{pfx}.ffn.norm1", dim)
    _conv1(out, f"{pfx}.ffn.project_in", dim, 2 * hidden, False)
    out.append((f"{pfx}.ffn.dwconv.weight", (2 * hidden, 1, 3, 3), "conv"))
    _conv1(out, f"{pfx}.ffn.project_out", hidden, dim, False)


def _cab(out, pfx, dim):
    _res_block(out, f"{pfx}.residual_trunk.0", dim)
    _res_block(out, f"{pfx}.residual_trunk.1", dim)
    _conv3(out, f"{pfx}.subscale", dim, dim)
    _res_block(out, f"{pfx}.residual_mask2.0", dim)
    _res_block(out, f"{pfx}.residual_mask3.0", dim)
    _conv_t(out, f"{pfx}.upscale", dim, dim, 3)


def _tam(out, pfx, dim, downsample):
    if downsample:
        _conv3(out, f"{pfx}.ds_conv", dim, dim)
        _conv_t(out, f"{pfx}.us_conv", dim, dim, 3)
    _transformer_block(out, f"{pfx}.TABs.0", dim)
    _transformer_block(out, f"{pfx}.TABs.1", dim)


def param_specs(op: str, component: str):
    """``[(name, shape, kind)]`` of one synthesis net; ``op`` in sop/bop/hop, ``component`` in
    y/uv. Layouts follow ``fuzz/fuzz_targets/common.rs:260-345``."""
    t: list = []
    key = (op.lower(), component.lower())
    if key == ("sop", "y"):
        _conv3(t, "first_stage.0.0.conv1", 160, 160)
        t.append(("first_stage.1.conv.weight", (256, 160, 2, 2), "conv"))
        _res_au(t, "first_stage.2", 64, 4)
        t.append(("conv2_t.conv.weight", (128, 64, 2, 2), "conv"))
        _res_au(t, "iact2", 32, 2)
        _conv3(t, "conv3", 32, 32)
        _res_au(t, "iact3", 32, 2)
        _conv1(t, "conv4", 32, 16, False)
    elif key == ("sop", "uv"):
        _conv3(t, "first_stage.conv1", 256, 48)
        t.append(("conv2_t.conv.weight", (128, 144, 2, 2), "conv"))
        _res_au(t, "iact2", 32, 2)
        _conv3(t, "conv3", 32, 32)
        _res_au(t, "iact3", 32, 2)
        _conv1(t, "conv4", 32, 128, False)
    elif key == ("bop", "y"):
        _conv3(t, "first_stage.0.0.conv1", 160, 160)
        _conv_t(t, "first_stage.1", 160, 64, 4)
        _res_au(t, "first_stage.2", 64, 4)
        _conv_t(t, "conv2_t", 64, 64, 4)
        _res_au(t, "iact2", 64, 4)
        _conv3(t, "conv3", 64, 96)
        _res_au(t, "iact3", 96, 6)
        _conv1(t, "conv4", 96, 16, False)
    elif key == ("bop", "uv"):
        _conv3(t, "first_stage.conv1", 256, 48)
        _conv_t(t, "conv2_t", 144, 64, 4)
        _res_au(t, "iact2", 64, 4)
        _conv3(t, "conv3", 64, 128)
        _res_au(t, "iact3", 128, 8)
        _conv1(t, "conv4", 128, 128, False)
    elif key == ("hop", "y"):
        c = 128
        _res_block(t, "first_stage.0.0", 160)
        _conv_t(t, "first_stage.1", 160, c, 3)
        _res_au(t, "first_stage.2", c, 4)
        _conv_t(t, "conv2_t", c, c, 3)
        _cab(t, "CAB", c)
        _res_au(t, "iact2", c, 4)
        _conv1(t, "conv3_t", c, 4 * c, True)
        _tam(t, "TAM", c, True)
        _res_au(t, "iact3", c, 4)
        _conv_t(t, "conv4_t", c, 1, 3)
    elif key == ("hop", "uv"):
        c = 64
        _conv3(t, "first_stage.conv1", 256, 48)
        _conv_t(t, "conv2_t", 144, c, 3)
        _cab(t, "CAB", c)
        _res_au(t, "iact2", c, 4)
        _conv1(t, "conv3_t", c, 4 * c, True)
        _tam(t, "TAM", c, False)
        _res_au(t, "iact3", c, 4)
        _conv_t(t, "conv4_t", c, 8, 3)
    else:
        raise ValueError(f"unknown net {op}/{component}")
    return t


def random_params(op: str, component: str, seed: int = 1, gain: float = 1.0,
                  out_gain: float | None = None) -> dict:
    """He-normal random-init parameters of one net, keyed by checkpoint name. ``gain`` scales
    every He std; ``out_gain`` (if given) replaces it for the net's last layer."""
    specs = param_specs(op, component)
    last_w = [n for n, _, k in specs if k in ("conv", "convt")][-1]
    params = {}
    for name, shape, kind in specs:
        if kind == "conv":
            fan_in = shape[1] * shape[2] * shape[3]
        elif kind == "convt":
            fan_in = shape[0] * (shape[2] / 2.0) ** 2
        if kind in ("conv", "convt"):
            g = out_gain if (out_gain is not None and name == last_w) else gain
            params[name] = normal(seed, f"{op}/{component}/{name}", shape,
                                  g * np.sqrt(2.0 / fan_in))
        elif kind == "bias":
            params[name] = normal(seed, f"{op}/{component}/{name}", shape, 0.01)
        elif kind == "ones":
            params[name] = np.ones(shape, np.float32)
        else:
            params[name] = np.zeros(shape, np.float32)
    return params


def f16_weights(params: dict) -> dict:
    """The reference's f16-weight semantics (src/weights/f16.rs:70-72 ``round_trip``, as a
    ``ZJB2`` bundle stores a synthesis net): every float tensor rounded to IEEE half (round to
    nearest even, subnormals kept, overflow to infinity) and widened back, for nets that still
    compute in f32."""
    return {k: np.asarray(v, np.float32).astype(np.float16).astype(np.float32) for k, v in params.items()}


# ---------------------------------------------------------------------------------------------
# Latent reconstruction networks (hyper-decoder + multi-stage context model) of one component.
# ---------------------------------------------------------------------------------------------

LATENT_CHANNELS = (160, 96)  # src/header.rs:31


def latent_param_specs(component: int, context: bool = True):
    """``[(name, shape, kind)]`` of a component's ``HyperDecoder`` (src/model/hyper_decoder.rs:
    24-45) and, with ``context``, its ``ContextModel`` (src/model/mcm.rs:123-159)."""
    c = LATENT_CHANNELS[component]
    t: list = []
    _conv1(t, "hyper_decoder.conv1", c, c, False)
    _conv_t(t, "hyper_decoder.conv2", c, c, 4)
    _conv3(t, "hyper_decoder.conv3", c, c)
    _conv3(t, "hyper_decoder.conv4", c, 4 * c)
    if context:
        for s in range(4):
            p = f"context.MCM.{s}"
            if s > 0:
                _conv1(t, f"{p}.conv.0", s * c, c, False)
                t.append((f"{p}.conv.1.weight", (c, 32, 3, 3), "conv"))
                t.append((f"{p}.conv.1.bias", (c,), "bias"))
            _conv1(t, f"{p}.fusion_pred_net.conv1", c if s == 0 else 2 * c, c, False)
            _conv1(t, f"{p}.fusion_pred_net.conv2", c, c, False)
            _conv1(t, f"{p}.fusion_pred_net.conv3", c, c, False)
    return t


def random_latent_params(component: int, seed: int = 1, gain: float = 1.0,
                         context: bool = True) -> dict:
    """He-normal random-init parameters of a component's latent reconstruction networks."""
    params = {}
    for name, shape, kind in latent_param_specs(component, context):
        tag = f"latent/{component}/{name}"
        if kind == "conv":
            params[name] = normal(seed, tag, shape, gain * np.sqrt(2.0 / (shape[1] * shape[2] * shape[3])))
        elif kind == "convt":
            params[name] = normal(seed, tag, shape, gain * np.sqrt(2.0 / (shape[0] * (shape[2] / 2.0) ** 2)))
        else:
            params[name] = normal(seed, tag, shape, 0.01)
    return params


def hyper_latent(seed: int, name: str, c: int, h: int, w: int, b: float = 1.5) -> np.ndarray:
    """int8 ``z_hat`` ``[c, h, w]``: ``round(Laplace(0, b))`` clamped to the int8 range."""
    return np.clip(latent(seed, name, c, h, w, b), -128, 127).astype(np.int8)


def residual(seed: int, name: str, c: int, h: int, w: int, b: float = 0.5) -> np.ndarray:
    """A dequantised residual ``[c, h, w]``: continuous Laplace(0, b) samples."""
    return laplace(seed, name, (c, h, w), b)


# ---------------------------------------------------------------------------------------------
# Analysis transforms (encoder side, src/model/analysis.rs).
# ---------------------------------------------------------------------------------------------

ANALYSIS_HIDDEN = 128  # src/model/analysis.rs:32


def analysis_param_specs(op: str, component: str):
    """``[(name, shape, kind)]`` of ``AnalysisPrimary`` / ``AnalysisSecondary``
    (src/model/analysis.rs:122-153, :230-290) for ``op`` in bop/hop; ResAU groups of 16
    channels, as the synthesis ResAUs."""
    c = ANALYSIS_HIDDEN
    luma = component == "y"
    t: list = []
    _conv3(t, "conv1", 1 if luma else 12, c)
    _res_au(t, "act1", c, c // 16)
    if op == "hop":
        _tam(t, "TAM", c, luma)
    _conv3(t, "conv2", c, c)
    _res_au(t, "act2", c, c // 16)
    if op == "hop":
        _cab(t, "cab", c)
    _conv3(t, "conv3", c, c)
    _res_au(t, "act3", c, c // 16)
    if luma:
        _conv3(t, "conv4", c, LATENT_CHANNELS[0])
        _conv1(t, "conv5", LATENT_CHANNELS[0], LATENT_CHANNELS[0], False)
    else:
        _conv1(t, "conv5", c, LATENT_CHANNELS[1], False)
    return t


def random_analysis_params(op: str, component: str, seed: int = 1, gain: float = 1.0) -> dict:
    """He-normal random-init parameters of one analysis transform, keyed by checkpoint name."""
    params = {}
    for name, shape, kind in analysis_param_specs(op, component):
        tag = f"analysis/{op}/{component}/{name}"
        if kind == "conv":
            params[name] = normal(seed, tag, shape, gain * np.sqrt(2.0 / (shape[1] * shape[2] * shape[3])))
        elif kind == "convt":
            params[name] = normal(seed, tag, shape, gain * np.sqrt(2.0 / (shape[0] * (shape[2] / 2.0) ** 2)))
        elif kind == "bias":
            params[name] = normal(seed, tag, shape, 0.01)
        elif kind == "ones":
            params[name] = np.ones(shape, np.float32)
        else:
            params[name] = np.zeros(shape, np.float32)
    return params


def picture(seed: int, name: str, c: int, h: int, w: int) -> np.ndarray:
    """Picture planes ``[c, h, w]`` in [0, 255] (uniform samples, whole numbers)."""
    return np.floor(uniform(seed, name, (c, h, w), 0.0, 256.0)).clip(0, 255).astype(np.float32)
