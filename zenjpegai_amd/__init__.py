"""zenjpegai_amd: MI355X (gfx950) HIP backend for the JPEG AI synthesis transform of
imazen/zenjpegai.

The product is ``libzjai_hip.so`` (HIP kernels + C-ABI, ``include/zjai_hip.h``); this package
holds its sources (``csrc/``) and a ctypes mirror of the reference's operator and model API:

* ``zenjpegai_amd.nn``    -- ``Engine``, ``Conv2d``/``ConvTranspose2d``, ``ConvLayer``,
  ``ConvTransposeLayer``, ``BTensor`` and the elementwise / attention ops;
* ``zenjpegai_amd.model`` -- ``SynthesisPrimary``, ``SynthesisSecondary``,
  ``synthesis_tiles``, ``Picture`` and ``synthesize``;
* ``zenjpegai_amd.synth`` -- seeded synthetic weights and latents.
"""

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))


def build(jobs: int = 8, force: bool = True) -> str:
    """Compiles ``libzjai_hip.so`` for gfx950 in-tree and returns its path; ``force`` rebuilds
    every object even where make finds it up to date."""
    cmd = ["make", "-s", f"-j{jobs}", "-C", os.path.join(HERE, "csrc")]
    if force:
        cmd.insert(1, "-B")
    subprocess.run(cmd, check=True)
    return os.path.join(HERE, "libzjai_hip.so")
