"""Measures the device buffer-pool use of whole-picture syntheses on an MI355X and writes it as
the fixture ``pool_use_mi355x.json`` beside this script (run from the repository root on a GPU
box: ``python3 tests/golden/pool_use.py [output path]``).

Per case (operating point, precision, picture size, tiling, chroma net or not, lane count): a
released context (``zjai_release_buffers``) runs one picture of the benchmark's random nets, then
``zjai_get_stats`` gives ``pool_peak`` (blocks in use at once, summed over the lanes' pools) and
``pool_cached`` (blocks the pools keep). ``tests/test_memory_estimate.py`` checks the device
memory estimate (``zjai_picture_estimate_memory``) against these figures on the CPU; the GPU test
``tests/test_gpu_memory.py`` measures other shapes live.
"""

import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from zenjpegai_amd import model, nn, synth  # noqa: E402

# height, width, tiling (size, overlap) or None, region grid or None, chroma net, lanes
SHAPES = [
    (256, 256, None, None, False, 1),
    (256, 256, None, None, True, 1),
    (512, 512, None, None, True, 1),
    (512, 768, None, None, True, 1),
    (1024, 1024, None, None, False, 1),
    (1024, 1024, None, None, True, 1),
    (1080, 1920, (512, 64), None, True, 1),
    (1080, 1920, (512, 64), None, True, 3),
    (2048, 2048, (1024, 64), None, True, 1),
    (2160, 3840, (640, 128), (2, 3), True, 1),
    (2160, 3840, (640, 128), (2, 3), True, 4),
]


def measure(prec, op, out):
    eng = nn.Engine(0, prec)
    prim = model.SynthesisPrimary.load(synth.random_params(op, "y", seed=1), op, eng)
    sec = model.SynthesisSecondary.load(synth.random_params(op, "uv", seed=1), op, eng)
    for h, w, tiling, regions, uv, lanes in SHAPES:
        if op != "hop" and h > 1100:
            continue
        lh, lw = -(-h // 16), -(-w // 16)
        tiles = model.synthesis_tiles(h, w, lh, lw, tiling, regions)
        eng.release_buffers()
        s = 2 if uv else 1
        pic = model.Picture(eng, prim, sec if uv else None, lh, lw, h, w, tiles, s, s,
                            bit_depth=10, lanes=lanes)
        pic.upload(synth.latent(1, "pool/y", 160, lh, lw),
                   synth.latent(1, "pool/uv", 96, lh, lw) if uv else None)
        pic.run()
        eng.sync()
        st = eng.stats()
        rec = dict(op=op, precision=prec, height=h, width=w, tiling=tiling, regions=regions,
                   uv=uv, lanes=lanes, pool_peak=st["pool_peak"], pool_cached=st["pool_cached"])
        print(json.dumps(rec), flush=True)
        out.append(rec)
        del pic
    del prim, sec
    eng.close()


def main():
    out = []
    for prec in ("f32", "bf16"):
        for op in ("sop", "bop", "hop"):
            measure(prec, op, out)
    path = sys.argv[1] if len(sys.argv) > 1 else os.path.join(
        os.path.dirname(os.path.abspath(__file__)), "pool_use_mi355x.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=0)
        f.write("\n")


if __name__ == "__main__":
    main()
