"""CPU restatement of the packed weight containers -- TEST INFRASTRUCTURE ONLY (imported by
``tests/`` as the checker, never by the product library).

``ZJM1`` checkpoints and ``ZJB1`` / ``ZJB2`` bundles as documented in
``src/weights/packed.rs:8-42``: little-endian tables, payloads at absolute offsets that are
multiples of 64, each payload zero-padded to a multiple of 64. Pure Python/numpy, written from
the format description (writer: ``write_zjm_impl`` :236-297, ``write_bundle_with`` :305-334;
reader: ``parse_zjm`` :150-205, ``PackedBundle::add`` :307-345).

Pinned by: a hand-assembled known-answer file (``tests/test_weights.py``), the layout
invariants (offsets and lengths multiples of 64, tables exactly as long as their entries), and
the round trip through the independent C++ reader and writer of the product library.
"""

from __future__ import annotations

import struct

import numpy as np

ALIGN = 64
VERSION = 1
# dtype codes of `dtype_code` (src/weights/packed.rs:62-75)
CODES = {"F64": 0, "F32": 1, "F16": 2, "I64": 3, "I32": 4, "I16": 5, "I8": 6, "U8": 7, "Bool": 8}
NP = {"F64": "<f8", "F32": "<f4", "F16": "<f2", "I64": "<i8", "I32": "<i4", "I16": "<i2",
      "I8": "i1", "U8": "u1", "Bool": "?"}
NAMES = {v: k for k, v in CODES.items()}
F16_KEEP_F32 = ("vr_vec.c",)  # src/weights/packed.rs:221


def _pad(b: bytearray) -> None:
    b.extend(b"\0" * (-len(b) % ALIGN))


def write_zjm(tensors, ints=(), f16=False) -> bytes:
    """tensors: [(name, dtype name, numpy array)], ints: [(name, int)]."""
    payloads = []
    for name, dt, arr in tensors:
        a = np.array(arr, dtype=NP[dt], order="C")  # keeps rank 0 (ascontiguousarray would not)
        if f16 and dt == "F32" and name not in F16_KEEP_F32:
            dt, a = "F16", a.astype("<f2")  # IEEE round to nearest even
        payloads.append((name, dt, a.shape, a.tobytes()))
    table = 16 + sum(2 + len(n.encode()) + 2 + 8 * len(s) + 16 for n, _, s, _ in payloads)
    table += sum(2 + len(n.encode()) + 8 for n, _ in ints)
    out = bytearray(b"ZJM1" + struct.pack("<III", VERSION, len(payloads), len(ints)))
    offset = table + (-table % ALIGN)
    for name, dt, shape, data in payloads:
        nb = name.encode()
        out += struct.pack("<H", len(nb)) + nb + struct.pack("<BB", CODES[dt], len(shape))
        out += b"".join(struct.pack("<Q", d) for d in shape)
        out += struct.pack("<QQ", offset, len(data))
        offset += len(data)
        offset += -offset % ALIGN
    for name, v in ints:
        nb = name.encode()
        out += struct.pack("<H", len(nb)) + nb + struct.pack("<q", v)
    assert len(out) == table
    _pad(out)
    for _, _, _, data in payloads:
        out += data
        _pad(out)
    return bytes(out)


def read_zjm(data: bytes):
    """(tensors {name: (dtype name, array)}, ints [(name, value)]); raises ValueError."""
    if data[:4] != b"ZJM1":
        raise ValueError("bad magic")
    version, nt, ni = struct.unpack_from("<III", data, 4)
    if version != VERSION:
        raise ValueError("unsupported version")
    pos, tensors, ints = 16, {}, []
    for _ in range(nt):
        (n,) = struct.unpack_from("<H", data, pos)
        name = data[pos + 2:pos + 2 + n].decode()
        pos += 2 + n
        code, rank = struct.unpack_from("<BB", data, pos)
        pos += 2
        if code not in NAMES or rank > 8:
            raise ValueError("bad dtype or rank")
        shape = struct.unpack_from(f"<{rank}Q", data, pos)
        pos += 8 * rank
        off, ln = struct.unpack_from("<QQ", data, pos)
        pos += 16
        dt = NAMES[code]
        size = int(np.prod(shape, dtype=np.int64)) * np.dtype(NP[dt]).itemsize
        if size != ln or off % ALIGN or off + ln > len(data):
            raise ValueError(f"tensor {name} has an invalid extent")
        tensors[name] = (dt, np.frombuffer(data, NP[dt], count=size // np.dtype(NP[dt]).itemsize,
                                           offset=off).reshape(shape))
    for _ in range(ni):
        (n,) = struct.unpack_from("<H", data, pos)
        name = data[pos + 2:pos + 2 + n].decode()
        (v,) = struct.unpack_from("<q", data, pos + 2 + n)
        pos += 2 + n + 8
        ints.append((name, v))
    return tensors, ints


def write_bundle(files, notice: str, f16=False) -> bytes:
    """files: [(relative path, bytes)]."""
    nb = notice.encode()
    table = 16 + len(nb) + sum(2 + len(p.encode()) + 16 for p, _ in files)
    out = bytearray((b"ZJB2" if f16 else b"ZJB1") + struct.pack("<III", VERSION, len(files), len(nb)))
    out += nb
    offset = table + (-table % ALIGN)
    for path, data in files:
        pb = path.encode()
        out += struct.pack("<H", len(pb)) + pb + struct.pack("<QQ", offset, len(data))
        offset += len(data)
        offset += -offset % ALIGN
    assert len(out) == table
    _pad(out)
    for _, data in files:
        out += data
        _pad(out)
    return bytes(out)


def read_bundle(data: bytes):
    """(notice, {path: bytes}, f16 flag); raises ValueError."""
    if data[:4] not in (b"ZJB1", b"ZJB2"):
        raise ValueError("bad magic")
    version, count, nlen = struct.unpack_from("<III", data, 4)
    if version != VERSION:
        raise ValueError("unsupported version")
    notice = data[16:16 + nlen].decode()
    pos, files = 16 + nlen, {}
    for _ in range(count):
        (n,) = struct.unpack_from("<H", data, pos)
        path = data[pos + 2:pos + 2 + n].decode()
        off, ln = struct.unpack_from("<QQ", data, pos + 2 + n)
        pos += 2 + n + 16
        if off % ALIGN or off + ln > len(data):
            raise ValueError(f"{path} has an invalid extent")
        files[path] = data[off:off + ln]
    return notice, files, data[:4] == b"ZJB2"
