"""Reader for the ZJTB layer fixtures copied from the reference's `tests/vectors/nn/`.

Format (as `tests/nn_vectors.rs:16-48` of the reference reads it): magic ``ZJTB``, u32 LE count,
then per array: u16 LE name length, UTF-8 name, u8 ndim, ndim x u32 LE dims, f32 LE data.
The fixtures were produced by PyTorch 1.10.2 (the reference's `scripts/ref_vectors/gen_nn_vectors.py`;
`bicubic_align_corners` / `bilinear_align_corners` by its `gen_resize_vectors.py`).
"""

import os
import struct

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def load(name: str) -> dict:
    with open(os.path.join(HERE, f"{name}.bin"), "rb") as f:
        b = f.read()
    assert b[:4] == b"ZJTB"
    pos = 4
    (count,) = struct.unpack_from("<I", b, pos)
    pos += 4
    out = {}
    for _ in range(count):
        (nlen,) = struct.unpack_from("<H", b, pos)
        pos += 2
        key = b[pos:pos + nlen].decode()
        pos += nlen
        ndim = b[pos]
        pos += 1
        shape = struct.unpack_from(f"<{ndim}I", b, pos)
        pos += 4 * ndim
        n = int(np.prod(shape))
        out[key] = np.frombuffer(b, "<f4", n, pos).reshape(shape).copy()
        pos += 4 * n
    assert pos == len(b)
    return out
