"""Benchmark of the MI355X synthesis path (one JSON line on stdout).

Workload (``config.workload``): BASELINE config 5 -- HOP luma + chroma synthesis of a 3840x2160
4:2:0 picture, 10-bit output, tiled as the reference's encoder signals it for independent
regions (2x3 regions, tile 640, overlap 128: 24 tiles), He-normal random-init weights, latents
round(Laplace(0, 1.5)) at /16 resolution. One step = one whole-picture synthesis with the
latents already resident in HBM (``Picture.run``: the tiles in same-shape batches of up to 6 over
``--lanes`` concurrent HIP streams, 4 by default; 10-bit planes written by the last layers'
epilogues).

``value`` is the fp32-MFMA parity path (the reference computes in f32) in replay mode: the
picture's launch sequence captured once as a HIP graph and launched again each step, as a
decoder of many pictures of one geometry runs it (the reference's GPU backend replays a dispatch
plan per tile geometry the same way). ``eager``: the same picture with every launch issued from
the host; ``one_stream``: eager with every launch on one HIP stream.

Extra lines in ``extra``: the host-to-host rate of the same picture (latent upload, synthesis,
download of the 10-bit planes; ``host_to_host``), the device time of the last timed step, the
same picture on the bf16 path and on the f16 path (the latter timed on He x 0.5 weights, whose
activations stay inside f16's range), eager and replayed (``*_replay_mpix_s``), with the PSNR of
their 10-bit planes against the f32 path's at gains 1 and 0.5, the number of f16 activations
stored as non-finite at both gains (``ZJAI_CTX_COUNT_F16_RANGE``), the reference's f16-weight
semantics (weights rounded to f16, f32 activations: time and PSNR at both gains), BASELINE
config 4 (SOP luma 1024x1024, 8-bit; f32 and bf16, eager and replayed), a 4 MP HOP picture
(2048x2048, 1 MP header tiles) and BASELINE configs 1-3 as single layers (kernel time and
TFLOP/s, f32 and bf16).

``roofline``: one profiled step (HIP events around every launch, all on one stream); the
dominant kernel is the one with the largest summed time; bound by its arithmetic intensity
against the machine balance; achieved = its algorithmic FLOPs (all taps, padding included) or
compulsory bytes / its summed time. ``traffic``: HBM bytes per launch of that kernel
from the rocprofv3 FETCH_SIZE / WRITE_SIZE passes summarised in ``profiles/`` (null if absent).

``cpu_baseline``: the reference's CPU engine ``nn::fast`` restated in C++ (``oracle/fast_cpu.cpp``,
bit-identical to the oracle) timed on a bounded sample of the same workload -- the config-5 tiles
in order for about 20 s, luma + chroma -- on this host's cores; plus the first tile on one thread,
the restatement's GMAC/s on a dense 3x3 160 -> 160 layer (one thread and all, beside the
reference's published one-thread figure) and the host CPU as lscpu reports it.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "synthesis decode Mpixel/s at 1MP & 4MP; conv TFLOP/s + % MFMA peak (1 GPU)"
PEAK_TFLOPS = {"f32": 157.3, "f16": 2500.0, "bf16": 2500.0}
PEAK_HBM_GBS = 8000.0
# The MFMA convolution kernels (conv.hip, conv32.hip, conv1x1.hip).
CONV_KERNELS = ("conv_igemm", "conv_dma_f32", "conv_tr_merged", "conv3x3_m32", "conv1x1_ring")


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def make_workload(name, eng, lanes=1, bits=None, gain=1.0, f16_weights=False):
    """``bits``: output bit depth override (0 = float planes); ``gain``: He-std scale of the
    random weights (1 = the benchmarked nets); ``f16_weights``: every weight rounded to f16 and
    back (the reference's f16-weight semantics) before the net is built."""
    from zenjpegai_amd import model, synth
    bits_override = bits
    if name == "cfg5":
        h, w, op, sv, sh, bits = 2160, 3840, "hop", 2, 2, 10
        lh, lw = 135, 240
        tiles = model.synthesis_tiles(h, w, lh, lw, (640, 128), (2, 3))
        uv = True
    elif name == "hop4mp":
        # 2048 x 2048 (4.19 MP), the reference's 4 MP sweep size; header tiling without
        # independent regions: 1 MP tiles (1024, overlap 64; src/encoder/tiles.rs:294-317).
        h, w, op, sv, sh, bits = 2048, 2048, "hop", 2, 2, 10
        lh, lw = 128, 128
        tiles = model.synthesis_tiles(h, w, lh, lw, (1024, 64))
        uv = True
    elif name == "cfg4":
        h, w, op, sv, sh, bits = 1024, 1024, "sop", 1, 1, 8
        lh, lw = 64, 64
        tiles = model.synthesis_tiles(h, w, lh, lw, None)
        uv = False
    else:
        raise SystemExit(f"unknown workload {name}")
    rnd = synth.f16_weights if f16_weights else (lambda p: p)
    py = rnd(synth.random_params(op, "y", seed=1, gain=gain))
    y = synth.latent(1, f"{name}/y", 160, lh, lw)
    prim = model.SynthesisPrimary.load(py, op, eng)
    sec, uvl, puv = None, None, None
    if uv:
        puv = rnd(synth.random_params(op, "uv", seed=1, gain=gain))
        sec = model.SynthesisSecondary.load(puv, op, eng)
        uvl = synth.latent(1, f"{name}/uv", 96, lh, lw)
    if bits_override is not None:
        bits = bits_override
    pic = model.Picture(eng, prim, sec, lh, lw, h, w, tiles, sv, sh, bit_depth=bits, lanes=lanes)
    pic.upload(y, uvl)
    return pic, dict(h=h, w=w, op=op, tiles=len(tiles), bits=bits, sv=sv, sh=sh,
                     latent=(lh, lw), py=py, y=y, uvl=uvl, puv=puv, tile_list=tiles)


def time_steps(eng, pic, steps, warmup):
    for _ in range(warmup):
        pic.run()
    eng.sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        pic.run()
    eng.sync()
    return (time.perf_counter() - t0) * 1e3 / steps


def host_to_host(eng, pic, info, reps):
    """One picture from latents on the host to quantised planes on the host: upload of y_hat and
    uv_hat (host -> HBM), the synthesis, download of the Y, U and V planes (HBM -> host), all
    synchronous, averaged over ``reps`` pictures after one warm-up. The host buffers are
    page-locked (``Engine.host_array``), as a caller decoding picture after picture keeps them;
    ``pageable_ms_per_picture`` is the same with ordinary numpy arrays."""
    def timed(y, uv, out):
        pic.upload(y, uv)
        pic.run()
        pic.download(out)
        t0 = time.perf_counter()
        for _ in range(reps):
            pic.upload(y, uv)
            pic.run()
            pic.download(out)
        return (time.perf_counter() - t0) * 1e3 / reps
    pageable = timed(info["y"], info["uvl"], None)
    y = eng.host_array(info["y"].shape)
    y[...] = info["y"]
    uv = None
    if info["uvl"] is not None:
        uv = eng.host_array(info["uvl"].shape)
        uv[...] = info["uvl"]
    dt = np.uint16 if pic.bit_depth else np.float32
    ch, cw = -(-pic.out_h // pic.sv), -(-pic.out_w // pic.sh)
    planes_uv = (eng.host_array((ch, cw), dt), eng.host_array((ch, cw), dt)) if uv is not None else (None, None)
    out = (eng.host_array((pic.out_h, pic.out_w), dt),) + planes_uv
    ms = timed(y, uv, out)
    return {"ms_per_picture": round(ms, 3), "mpix_s": round(info["h"] * info["w"] / (ms / 1e3) / 1e6, 3),
            "pageable_ms_per_picture": round(pageable, 3)}


def plane_psnr(ref, got, bits):
    """PSNR (dB) of each output plane against the f32 path's, at the planes' bit depth."""
    peak = float((1 << bits) - 1) if bits else 255.0
    out = {}
    for name, a, b in zip("yuv", ref, got):
        if a is None:
            continue
        mse = float(np.mean((a.astype(np.float64) - b.astype(np.float64)) ** 2))
        out[name] = round(10.0 * np.log10(peak * peak / mse), 2) if mse > 0 else None
    return out


def profile_step(eng, pic):
    """One step on a single stream with HIP events around every launch (concurrent lanes would
    overlap kernels and inflate each one's event-measured duration)."""
    lanes = pic.lanes
    pic.set_lanes(1)
    eng.profile_begin()
    pic.run()
    recs = eng.profile_end()
    pic.set_lanes(lanes)
    by = {}
    for name, flops, nbytes, ms in recs:
        d = by.setdefault(name, {"count": 0, "ms": 0.0, "flops": 0.0, "bytes": 0.0})
        d["count"] += 1
        d["ms"] += ms
        d["flops"] += flops
        d["bytes"] += nbytes
    return by


def rgb_output_stage(prec, lanes, reps=5):
    """The decoder's output stage for a BT.709 stream on the config-5 picture (float planes):
    bicubic 4:2:0 -> 4:4:4 chroma, BT.709 -> RGB, clip, 10-bit quantisation, one kernel.
    Kernel time from HIP events (best of ``reps``); bytes are the luma read, the chroma planes
    read once and the interleaved uint16 RGB written."""
    from zenjpegai_amd import nn
    eng = nn.Engine(0, prec)
    pic, info = make_workload("cfg5", eng, lanes, bits=0)
    pic.run()
    best = None
    for _ in range(reps):
        eng.profile_begin()
        pic.download_rgb(10)
        recs = [r for r in eng.profile_end() if r[0] == "k_picture_rgb"]
        best = recs[0] if best is None or recs[0][3] < best[3] else best
    n = info["h"] * info["w"]
    nbytes = n * (4 + 6) + 2 * 4 * (-(-info["h"] // 2)) * (-(-info["w"] // 2))
    us = best[3] * 1e3
    return {"kernel_us": round(us, 2), "algorithmic_GB_s": round(nbytes / (us * 1e-6) / 1e9, 1),
            "mpix_s": round(n / (us * 1e-6) / 1e6, 1)}


def latent_stage(prec, reps=3):
    """The decoder's latent reconstruction of the config-5 picture (2x3 independent regions,
    src/decoder/reconstruct.rs:81-234): per component the hyper-decoder on every region's z
    window and the four-stage context model on its residual / psi windows, one
    ``zjai_reconstruct_latent`` call each. Reports the summed kernel time (HIP events, best of
    ``reps``), the call's wall time (host transfers of z_hat, residual, psi and y_hat included)
    and the algorithmic FLOPs; returns the inputs for the CPU leg."""
    from zenjpegai_amd import model, nn, synth
    eng = nn.Engine(0, prec)
    regions = model.Regions(2, 3, True)
    out, inputs = {}, []
    for ccs, tag in ((0, "luma"), (1, "chroma")):
        c = synth.LATENT_CHANNELS[ccs]
        p = synth.random_latent_params(ccs, seed=1)
        m = model.LatentModel.load(p, ccs, eng)
        z = synth.hyper_latent(1, f"cfg5/z{ccs}", c, 34, 60)
        res = synth.residual(1, f"cfg5/r{ccs}", c, 135, 240)
        m.reconstruct(2160, 3840, regions, z, res)
        best_k, best_w, flops = None, None, 0.0
        for _ in range(reps):
            eng.profile_begin()
            t0 = time.perf_counter()
            m.reconstruct(2160, 3840, regions, z, res)
            wall = (time.perf_counter() - t0) * 1e3
            recs = eng.profile_end()
            k = sum(r[3] for r in recs)
            flops = sum(r[1] for r in recs)
            best_k = k if best_k is None else min(best_k, k)
            best_w = wall if best_w is None else min(best_w, wall)
        out[f"{tag}_kernel_ms"] = round(best_k, 3)
        out[f"{tag}_wall_ms"] = round(best_w, 3)
        out[f"{tag}_gflop"] = round(flops / 1e9, 2)
        inputs.append((ccs, p, z, res))
        del m
    eng.close()
    return out, inputs


def latent_stage_cpu(inputs):
    """The same latent reconstruction on the CPU restatement (nn::fast convolutions)."""
    import oracle.graphs as og
    from oracle import geometry as geo
    out = {}
    for ccs, p, z, res in inputs:
        t0 = time.perf_counter()
        with og.fast_convs():
            og.reconstruct_latent(p, ccs, 2160, 3840, geo.Regions(2, 3, True), z, res)
        out[("luma" if ccs == 0 else "chroma") + "_cpu_ms"] = round((time.perf_counter() - t0) * 1e3, 1)
    return out


def analysis_stage(prec, reps=3):
    """The encoder's analysis transforms (src/model/analysis.rs) on the config-5 picture: HOP
    primary on the 3840x2160 luma plane and HOP secondary on the 12 half-resolution planes, one
    ``zjai_analysis_forward`` call each. Reports the summed kernel time (HIP events, best of
    ``reps``), the wall time (host transfers included), the algorithmic FLOPs and the picture's
    Mpixel/s over the kernel time of both."""
    from zenjpegai_amd import model, nn, synth
    eng = nn.Engine(0, prec)
    out, total = {}, 0.0
    for comp, cls, planes, h, w in (("y", model.AnalysisPrimary, 1, 2160, 3840),
                                    ("uv", model.AnalysisSecondary, 12, 1080, 1920)):
        net = cls.load(synth.random_analysis_params("hop", comp, seed=1), "hop", eng)
        x = synth.picture(1, f"cfg5/analysis/{comp}", planes, h, w)
        net.forward(eng, x)
        best_k, best_w, flops = None, None, 0.0
        for _ in range(reps):
            eng.profile_begin()
            t0 = time.perf_counter()
            net.forward(eng, x)
            wall = (time.perf_counter() - t0) * 1e3
            recs = eng.profile_end()
            k = sum(r[3] for r in recs)
            flops = sum(r[1] for r in recs)
            best_k = k if best_k is None else min(best_k, k)
            best_w = wall if best_w is None else min(best_w, wall)
        out[f"{comp}_kernel_ms"] = round(best_k, 3)
        out[f"{comp}_wall_ms"] = round(best_w, 3)
        out[f"{comp}_gflop"] = round(flops / 1e9, 1)
        out[f"{comp}_tflops"] = round(flops / (best_k / 1e3) / 1e12, 1)
        total += best_k
        del net
    out["mpix_s"] = round(3840 * 2160 / (total / 1e3) / 1e6, 1)
    eng.close()
    return out


def layer_configs(prec, reps=10):
    """BASELINE configs 1-3 as single-layer runs at their full sizes: kernel time per run (HIP
    events around each launch) and conv TFLOP/s (all taps counted)."""
    from zenjpegai_amd import _lib, nn, synth
    eng = nn.Engine(0, prec)
    he = lambda seed, name, shape, fan: synth.normal(seed, name, shape, float(np.sqrt(2.0 / fan)))
    x1 = nn.BTensor.from_planar(eng, synth.uniform(1, "cfg1/x", (128, 256, 256), -1, 1))
    c1 = nn.ConvLayer(nn.Conv2d(128, 128, (3, 3), 1, (1, 1), 1, he(1, "cfg1/w", (128, 128, 3, 3), 1152),
                                synth.normal(1, "cfg1/b", (128,), 0.01)), eng)
    x2 = nn.BTensor.from_planar(eng, synth.laplace(2, "cfg2/x", (192, 64, 64), 1.0))
    c2 = nn.ConvTransposeLayer(nn.ConvTranspose2d(192, 128, 4, 2, 1, 0, he(2, "cfg2/w", (192, 128, 4, 4), 768),
                                                  synth.normal(2, "cfg2/b", (128,), 0.01)), eng)
    x3 = nn.BTensor.from_planar(eng, synth.uniform(3, "cfg3/x", (192, 128, 128), -2, 2))
    mk = lambda k, name: nn.ConvLayer(nn.Conv2d(192, 192, (k, k), 1, (k // 2, k // 2), 1,
                                                he(3, f"cfg3/{name}w", (192, 192, k, k), 192 * k * k),
                                                synth.normal(3, f"cfg3/{name}b", (192,), 0.01)), eng)
    t1, t2, gt = mk(3, "c1"), mk(3, "c2"), mk(1, "g")

    def cfg3():
        # t = conv3x3(leaky(conv3x3(x))) + x; out = t * sigmoid(conv1x1(x)), epilogues fused.
        t = t1.forward_fused(eng, x3, act=_lib.ACT_LEAKY_RELU)
        t = t2.forward_fused(eng, t, res=_lib.RES_ADD, r1=x3)
        return gt.forward_fused(eng, x3, act=_lib.ACT_SIGMOID, res=_lib.RES_MUL, r1=t)

    runs = {"cfg1_conv3x3_128_256sq": lambda: c1.forward(eng, x1),
            "cfg2_convT4_192to128_leaky": lambda: c2.forward_fused(eng, x2, act=_lib.ACT_LEAKY_RELU),
            "cfg3_res_attn_block_192_128sq": cfg3}
    out = {}
    for key, fn in runs.items():
        for _ in range(3):
            fn()
        eng.sync()
        eng.profile_begin()
        for _ in range(reps):
            fn()
        recs = eng.profile_end()
        ms = sum(r[3] for r in recs)
        fl = sum(r[1] for r in recs)
        out[f"{key}_{prec}_us"] = round(ms * 1e3 / reps, 2)
        out[f"{key}_{prec}_tflops"] = round(fl / (ms / 1e3) / 1e12, 2)
    return out


def read_traffic(kernel, workload, precision):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    summary (``profiles/traffic_<workload>_<precision>.md``, lines
    ``TRAFFIC <workload> <precision> <bytes> <kernel>``), or None."""
    path = os.path.join(ROOT, "profiles", f"traffic_{workload}_{precision}.md")
    try:
        with open(path) as f:
            for line in f:
                parts = line.split(None, 4)
                if len(parts) == 5 and parts[0] == "TRAFFIC" and parts[1] == workload \
                        and parts[2] == precision and parts[4].strip() == kernel:
                    return float(parts[3])
    except OSError:
        pass
    return None


def cpu_host():
    """The host CPU as lscpu reports it: model, sockets, physical cores and logical CPUs (all on
    the machine), and the CPUs this process may use."""
    model, sockets, cores = None, set(), set()
    try:
        phys = None
        with open("/proc/cpuinfo") as f:
            for line in f:
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k == "model name" and model is None:
                    model = v
                elif k == "physical id":
                    phys = v
                    sockets.add(v)
                elif k == "core id":
                    cores.add((phys, v))
    except OSError:
        pass
    return {"model": model, "sockets": len(sockets) or None, "physical_cores": len(cores) or None,
            "logical_cpus": os.cpu_count(), "usable_cpus": len(os.sched_getaffinity(0))}


def cpu_conv_anchor(threads, reps=3):
    """GMAC/s of the nn::fast restatement on a dense 3x3 160 -> 160 layer at 107 x 107 positions
    (the reference's per-core anchor: res_conv3x3_160_160@1/16, 97.3 G ops/s on one thread of its
    AVX-512 tier, benchmarks/conv_kernels_2026-09-17.log:88-91)."""
    import oracle
    from zenjpegai_amd import synth
    oracle.set_cpu_threads(threads)
    x = synth.normal(1, "cpu/x", (160, 107, 107), 1.0)
    w = synth.normal(1, "cpu/w", (160, 160, 3, 3), 0.02)
    oracle.conv2d(x, w, None, 1, (1, 1), fast=True)
    t0 = time.perf_counter()
    for _ in range(reps):
        oracle.conv2d(x, w, None, 1, (1, 1), fast=True)
    dt = (time.perf_counter() - t0) / reps
    return round(107 * 107 * 160 * 160 * 9 / dt / 1e9, 1)


def cpu_tiles(info, budget_s, max_tiles=None):
    """Config-5 tiles in order through the CPU restatement until ``budget_s`` is spent: (tiles
    done, core pixels, seconds)."""
    import oracle.graphs as og
    done, pix, t0 = 0, 0, time.perf_counter()
    with og.fast_convs():
        for t in info["tile_list"]:
            lat = t.latent
            y = np.ascontiguousarray(info["y"][:, lat.y:lat.y + lat.height, lat.x:lat.x + lat.width])
            og.primary(info["py"], info["op"], y, t.image.height, t.image.width)
            if info["puv"] is not None:
                uv = np.ascontiguousarray(info["uvl"][:, lat.y:lat.y + lat.height, lat.x:lat.x + lat.width])
                og.secondary(info["puv"], info["op"], y, uv, t.image.height, t.image.width)
            done += 1
            pix += min(t.core.width, max(info["w"] - t.core.x, 0)) * min(t.core.height, max(info["h"] - t.core.y, 0))
            if time.perf_counter() - t0 >= budget_s or (max_tiles and done >= max_tiles):
                break
    return done, pix, time.perf_counter() - t0


def cpu_baseline(info, budget_s=20.0):
    """The CPU column: the reference's ``nn::fast`` engine restated in C++ (``oracle/fast_cpu.cpp``:
    NCHWc blocks, packed weights, im2col rows, AVX-512 24x16 FMA register tiles, OpenMP over
    rows; the rest of the graph on the oracle's C++ loops), run over the config-5 tiles in order
    until ``budget_s`` is spent. Rate = displayed (core) pixels of the finished tiles / time, the
    unit of ``value``."""
    import oracle
    threads = oracle.cpu_threads()
    done, pix, dt = cpu_tiles(info, budget_s)
    # One thread on the first tile (the per-core rate), then the threads restored.
    oracle.set_cpu_threads(1)
    d1, p1, t1 = cpu_tiles(info, 0.0, max_tiles=1)
    gmac1 = cpu_conv_anchor(1)
    oracle.set_cpu_threads(threads)
    gmac = cpu_conv_anchor(threads)
    tier = oracle.lib().fc_block_size()
    return {"value": round(pix / dt / 1e6, 4), "unit": "Mpixel/s", "cores": threads,
            "kind": "port",
            "sample": (f"{done} of {len(info['tile_list'])} tiles of the config-5 picture (HOP Y+UV, "
                       f"{pix / 1e6:.2f} MP of cores) through a C++ restatement of the reference's "
                       f"nn::fast engine ({'AVX-512' if tier == 16 else 'AVX2'} tier; convolutions "
                       f"blocked / row-vectorised, the other ops OpenMP loops), {dt:.1f} s"),
            "seconds": round(dt, 2),
            "one_thread": {"value": round(p1 / t1 / 1e6, 4), "unit": "Mpixel/s",
                           "sample": f"tile 0 ({p1 / 1e6:.3f} MP of core), {t1:.1f} s"},
            "conv3x3_160_gmac_s": {"threads_1": gmac1, f"threads_{threads}": gmac,
                                   "reference_threads_1": 97.3},
            "host": cpu_host()}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="cfg5", choices=["cfg5", "cfg4", "hop4mp"])
    ap.add_argument("--precision", default="f32", choices=["f32", "f16", "bf16"])
    ap.add_argument("--lanes", type=int, default=4,
                    help="concurrent streams the picture's tile batches run on (1 = one stream)")
    ap.add_argument("--no-extra", action="store_true", help="skip the extra precision / cfg4 runs")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--profile-out", default=None, help="write the per-kernel profile (JSON)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB (k_copy) 5 times: the known-size "
                         "kernel that calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE")
    args = ap.parse_args()
    if args.copy_probe:
        import numpy as np
        from zenjpegai_amd import nn
        eng = nn.Engine(0, "f32")
        c, w = 64, 1024
        h = args.copy_probe * (1 << 20) // (c * w * 4)
        t = nn.BTensor.zeros(eng, c, h, w)
        for _ in range(5):
            nn.BTensor.cat([t])
        eng.sync()
        print(json.dumps({"copy_probe_bytes_read": c * h * w * 4, "copy_probe_bytes_written": c * h * w * 4,
                          "kernel": "k_copy", "dispatches": 5}))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only; the synthesis tiles would shard "
              "across GPUs with no collective (each GPU runs whole tiles and writes its core "
              "rectangles), but no multi-GPU figure is produced.", file=sys.stderr)
        sys.exit(2)

    from zenjpegai_amd import nn

    eng = nn.Engine(0, args.precision)
    log(f"[bench] building workload {args.workload} ({args.precision})")
    pic, info = make_workload(args.workload, eng, args.lanes)
    log(f"[bench] {info['tiles']} tiles; warmup {args.warmup}, timing {args.steps} steps")
    # Eager runs: every launch issued from the host, batches over the lanes.
    ms_eager = time_steps(eng, pic, args.steps, args.warmup)
    pixels = info["h"] * info["w"]
    eager = {"lanes": args.lanes, "ms_per_step": round(ms_eager, 3), "value": round(pixels / (ms_eager / 1e3) / 1e6, 3)}
    log(f"[bench] eager: {ms_eager:.2f} ms/step -> {eager['value']:.2f} Mpixel/s")
    # The same picture with every kernel on the context's one stream (no concurrent lanes).
    pic.set_lanes(1)
    ms_one = time_steps(eng, pic, args.steps, args.warmup)
    pic.set_lanes(args.lanes)
    one_stream = {"lanes": 1, "ms_per_step": round(ms_one, 3), "value": round(pixels / (ms_one / 1e3) / 1e6, 3)}
    log(f"[bench] one stream: {ms_one:.2f} ms/step -> {one_stream['value']:.2f} Mpixel/s")
    # The headline: replay mode (the same lanes; the picture's launch sequence captured once as a
    # HIP graph and launched again each step, as a decoder of many pictures of one geometry runs
    # it). Same bytes as the eager runs (tests/test_gpu_replay.py).
    pic.set_replay(True)
    ms = time_steps(eng, pic, args.steps, args.warmup)
    last_step_device_ms = eng.stats()["last_run_ms"]
    pic.set_replay(False)
    value = pixels / (ms / 1e3) / 1e6
    log(f"[bench] replayed: {ms:.2f} ms/step -> {value:.2f} Mpixel/s")
    h2h = host_to_host(eng, pic, info, args.steps)
    log(f"[bench] host to host: {h2h}")
    planes_ref = pic.download() if args.precision == "f32" else None
    prof = profile_step(eng, pic)
    total_ms = sum(d["ms"] for d in prof.values())
    conv = {k: d for k, d in prof.items() if k.startswith(CONV_KERNELS)}
    conv_flops = sum(d["flops"] for d in conv.values())
    conv_ms = sum(d["ms"] for d in conv.values())
    dom_name, dom = max(prof.items(), key=lambda kv: kv[1]["ms"])
    # Bound by arithmetic intensity against the machine balance (peak FLOP/s / peak bytes/s):
    # below it the kernel is priced against HBM bandwidth, above it against the MFMA peak.
    balance = PEAK_TFLOPS[args.precision] * 1e12 / (PEAK_HBM_GBS * 1e9)
    if dom["flops"] > 0 and dom["bytes"] > 0 and dom["flops"] / dom["bytes"] >= balance:
        ach = dom["flops"] / (dom["ms"] / 1e3) / 1e12
        peak = PEAK_TFLOPS[args.precision]
        roof = {"bound": "mfma", "achieved": round(ach, 3), "peak": peak, "unit": "TFLOP/s"}
    else:
        ach = dom["bytes"] / (dom["ms"] / 1e3) / 1e9
        peak = PEAK_HBM_GBS
        roof = {"bound": "hbm", "achieved": round(ach, 1), "peak": peak, "unit": "GB/s"}
    roof["frac"] = round(ach / peak, 4)
    roof["traffic"] = read_traffic(dom_name, args.workload, args.precision)
    roof["kernel"] = dom_name
    roof["launches"] = dom["count"]
    roof["avg_launch_us"] = round(dom["ms"] * 1e3 / dom["count"], 2)
    roof["algorithmic_per_launch"] = round((dom["flops"] or dom["bytes"]) / dom["count"], 1)
    if args.profile_out:
        with open(args.profile_out, "w") as f:
            json.dump({"workload": args.workload, "precision": args.precision, "kernels": prof},
                      f, indent=1, sort_keys=True)

    latent_inputs = None
    extra = {
        "last_timed_step_device_ms": round(last_step_device_ms, 3),
        "host_to_host": h2h,
        "profiled_kernel_ms": round(total_ms, 3),
        "conv_tflops": round(conv_flops / (conv_ms / 1e3) / 1e12, 3) if conv_ms else None,
        "conv_frac_of_peak": round(conv_flops / (conv_ms / 1e3) / 1e12 / PEAK_TFLOPS[args.precision], 4) if conv_ms else None,
        "conv_share_of_kernel_time": round(conv_ms / total_ms, 4) if total_ms else None,
        "launches_per_step": sum(d["count"] for d in prof.values()),
    }
    if not args.no_extra:
        from zenjpegai_amd import _lib
        for prec in ("bf16", "f16"):
            if prec == args.precision:
                continue
            # f16 activations overflow on the gain-1 nets (their activations reach ~1e5, beyond
            # 65504: counted below), so the f16 path is timed on the He x 0.5 nets, where it
            # stays in range; the kernels and their launch sequence are the same.
            gain = 0.5 if prec == "f16" else 1.0
            e2 = nn.Engine(0, prec)
            p2, _ = make_workload(args.workload, e2, args.lanes, gain=gain)
            ms2 = time_steps(e2, p2, args.steps, args.warmup)
            pr2 = profile_step(e2, p2)
            cv = {k: d for k, d in pr2.items() if k.startswith(CONV_KERNELS)}
            cf, cm = sum(d["flops"] for d in cv.values()), sum(d["ms"] for d in cv.values())
            extra[f"{args.workload}_{prec}_mpix_s"] = round(pixels / (ms2 / 1e3) / 1e6, 3)
            extra[f"{args.workload}_{prec}_weights_he_gain"] = gain
            extra[f"{args.workload}_{prec}_conv_tflops"] = round(cf / (cm / 1e3) / 1e12, 3)
            p2.set_replay(True)
            ms2r = time_steps(e2, p2, args.steps, args.warmup)
            extra[f"{args.workload}_{prec}_replay_mpix_s"] = round(pixels / (ms2r / 1e3) / 1e6, 3)
            log(f"[bench] {prec}: {ms2:.2f} ms/step, replayed {ms2r:.2f} (He x {gain})")
            del p2, e2
        if args.precision == "f32" and args.workload == "cfg5":
            # PSNR of the 16-bit paths against the f32 planes on the benchmarked nets (gain 1)
            # and on better-conditioned ones (He x 0.5); the f16 runs count the f16 activations
            # stored non-finite (ZJAI_CTX_COUNT_F16_RANGE). Then the reference's own f16-weight
            # semantics: weights rounded to f16, activations and arithmetic f32.
            ref_e = nn.Engine(0, "f32")
            ref_p, _ = make_workload(args.workload, ref_e, args.lanes, gain=0.5)
            ref_p.run()
            ref_planes = {1.0: planes_ref, 0.5: ref_p.download()}
            del ref_p, ref_e
            suffix = {1.0: "", 0.5: "_he_x0.5"}
            nonfinite = {}
            for prec in ("bf16", "f16"):
                for gain in (1.0, 0.5):
                    e5 = nn.Engine(0, prec, _lib.CTX_COUNT_F16_RANGE if prec == "f16" else 0)
                    p5, _ = make_workload(args.workload, e5, args.lanes, gain=gain)
                    p5.run()
                    extra[f"{args.workload}_{prec}_psnr_db_vs_f32{suffix[gain]}"] = plane_psnr(
                        ref_planes[gain], p5.download(), info["bits"])
                    if prec == "f16":
                        nonfinite[f"he_x{gain:g}"] = int(e5.stats()["f16_nonfinite"])
                    del p5, e5
            extra[f"{args.workload}_f16_nonfinite_activations"] = nonfinite
            f16w = {}
            for gain in (1.0, 0.5):
                e6 = nn.Engine(0, "f32")
                p6, _ = make_workload(args.workload, e6, args.lanes, gain=gain, f16_weights=True)
                if gain == 1.0:
                    ms6 = time_steps(e6, p6, args.steps, args.warmup)
                    f16w["mpix_s"] = round(pixels / (ms6 / 1e3) / 1e6, 3)
                p6.run()
                f16w[f"psnr_db_vs_f32{suffix[gain]}"] = plane_psnr(ref_planes[gain], p6.download(), info["bits"])
                del p6, e6
            extra[f"{args.workload}_f16_weights_f32_activations"] = f16w
            log(f"[bench] f16 non-finite activations: {nonfinite}; f16 weights / f32 activations: {f16w}")
            log("[bench] PSNR vs f32: " + ", ".join(f"{k}={v}" for k, v in extra.items() if "psnr" in k))
        if args.workload != "cfg4":
            for prec in (args.precision, "bf16"):
                e3 = nn.Engine(0, prec)
                p3, i3 = make_workload("cfg4", e3, args.lanes)
                ms3 = time_steps(e3, p3, max(args.steps, 10), args.warmup)
                extra[f"cfg4_sop_1mp_{prec}_mpix_s"] = round(i3["h"] * i3["w"] / (ms3 / 1e3) / 1e6, 3)
                extra[f"cfg4_sop_1mp_{prec}_ms"] = round(ms3, 4)
                # Replay mode: the picture's launches captured once as a HIP graph.
                p3.set_replay(True)
                ms3r = time_steps(e3, p3, max(args.steps, 10), args.warmup)
                extra[f"cfg4_sop_1mp_{prec}_replay_ms"] = round(ms3r, 4)
                log(f"[bench] cfg4 {prec}: {ms3:.3f} ms/step, replayed {ms3r:.3f}")
                del p3, e3
        if args.workload == "cfg5":
            for prec in (args.precision, "bf16"):
                e4 = nn.Engine(0, prec)
                p4, i4 = make_workload("hop4mp", e4, args.lanes)
                ms4 = time_steps(e4, p4, args.steps, args.warmup)
                extra[f"hop_4mp_2048sq_{prec}_mpix_s"] = round(i4["h"] * i4["w"] / (ms4 / 1e3) / 1e6, 3)
                log(f"[bench] hop 4 MP {prec}: {ms4:.2f} ms/step")
                del p4, e4
        if args.workload == "cfg5":
            extra["rgb_output_stage_cfg5"] = rgb_output_stage(args.precision, args.lanes)
            log(f"[bench] RGB output stage: {extra['rgb_output_stage_cfg5']}")
            extra["latent_reconstruction_cfg5"], latent_inputs = latent_stage(args.precision)
            log(f"[bench] latent reconstruction: {extra['latent_reconstruction_cfg5']}")
            for prec in (args.precision, "bf16"):
                extra[f"analysis_hop_cfg5_{prec}"] = analysis_stage(prec)
                log(f"[bench] analysis transforms {prec}: {extra[f'analysis_hop_cfg5_{prec}']}")
        for prec in ("f32", "bf16"):
            extra.update(layer_configs(prec))
        log("[bench] configs 1-3: " + ", ".join(f"{k}={v}" for k, v in extra.items() if k.startswith("cfg") and "tflops" in k))

    cpu = None
    if not args.no_cpu:
        log("[bench] timing the CPU baseline (nn::fast restatement) on the config-5 tiles")
        cpu = cpu_baseline(info)
        log(f"[bench] cpu: {cpu}")
        if latent_inputs:
            extra["latent_reconstruction_cfg5"].update(latent_stage_cpu(latent_inputs))
            log(f"[bench] latent reconstruction with cpu: {extra['latent_reconstruction_cfg5']}")

    out = {
        "metric": METRIC, "value": round(value, 3), "unit": "Mpixel/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 3),
        "eager": eager,
        "one_stream": one_stream,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": args.precision, "data": "synthetic (He-normal random-init weights, Laplace latents)",
        "config": {
            "workload": {
                "cfg5": "cfg5: HOP Y+UV synthesis 3840x2160 4:2:0 10-bit, 2x3 independent regions, "
                        "tile 640 / overlap 128 (24 tiles), latents resident in HBM",
                "cfg4": "cfg4: SOP luma synthesis 1024x1024 8-bit, untiled, latent resident",
                "hop4mp": "HOP Y+UV synthesis 2048x2048 4:2:0 10-bit, tile 1024 / overlap 64, "
                          "latents resident in HBM"}[args.workload],
            "lanes": args.lanes,
            "mode": "replay: the whole picture's launches as one HIP graph (zjai_picture_set_replay); "
                    "eager: every launch from the host",
            "picture": f"{info['w']}x{info['h']}", "tiles": info["tiles"],
            "precision_path": args.precision},
        "roofline": roof,
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
