"""Weight readers over the C-ABI (host only, no GPU needed): PyTorch ``.pth`` checkpoints and
the packed ``ZJM1`` checkpoints / ``ZJB1`` / ``ZJB2`` bundles (``src/weights/mod.rs``,
``src/weights/packed.rs``). Names and behaviour follow the reference's ``Checkpoint`` and
``PackedBundle``; a ``Checkpoint`` feeds the synthesis and latent model loaders directly
(``SynthesisPrimary.load(ck, op, eng)``)."""

from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from ._lib import check, lib

# ZJM1 dtype codes (src/weights/packed.rs:62-75) -> (name, numpy dtype)
DTYPES = {
    0: ("F64", np.dtype("<f8")),
    1: ("F32", np.dtype("<f4")),
    2: ("F16", np.dtype("<f2")),
    3: ("I64", np.dtype("<i8")),
    4: ("I32", np.dtype("<i4")),
    5: ("I16", np.dtype("<i2")),
    6: ("I8", np.dtype("i1")),
    7: ("U8", np.dtype("u1")),
    8: ("Bool", np.dtype("?")),
}
MAX_RANK = 8


def _name(fn, *args) -> str:
    cap = 256
    while True:
        buf = ctypes.create_string_buffer(cap)
        rc = fn(*args, buf, cap)
        if rc == _lib.E_LIMIT and cap < 1 << 20:
            cap *= 4
            continue
        check(rc)
        return buf.value.decode()


class Checkpoint:
    """``Checkpoint::parse`` (src/weights/mod.rs:135): a ``.pth`` file or a packed ``ZJM1``
    file, told apart by the magic. Parsing never executes anything from the file."""

    def __init__(self, data: bytes):
        self._h = ctypes.c_void_p()
        check(lib().zjai_checkpoint_parse(data, len(data), ctypes.byref(self._h)))
        nt, ni, nl, packed = (ctypes.c_int32() for _ in range(4))
        check(lib().zjai_checkpoint_counts(self._h, ctypes.byref(nt), ctypes.byref(ni),
                                           ctypes.byref(nl), ctypes.byref(packed)))
        self._nt, self._ni, self._nl = nt.value, ni.value, nl.value
        self.packed = bool(packed.value)

    @classmethod
    def parse(cls, data: bytes) -> "Checkpoint":
        return cls(bytes(data))

    @classmethod
    def open(cls, path) -> "Checkpoint":
        with open(path, "rb") as f:
            return cls(f.read())

    @property
    def handle(self):
        return self._h

    def tensor_names(self) -> list[str]:
        return [_name(lib().zjai_checkpoint_tensor_name, self._h, i) for i in range(self._nt)]

    def contains(self, name: str) -> bool:
        return self.info(name) is not None

    def info(self, name: str):
        """(dtype name, shape) of a tensor, or None when absent."""
        dt, rank = ctypes.c_int32(), ctypes.c_int32()
        shape = (ctypes.c_int64 * MAX_RANK)()
        rc = lib().zjai_checkpoint_info(self._h, name.encode(), ctypes.byref(dt), ctypes.byref(rank),
                                        shape)
        if rc == _lib.E_MODEL:
            return None
        check(rc)
        return DTYPES[dt.value][0], tuple(shape[:rank.value])

    def _dtype_shape(self, name):
        dt, rank = ctypes.c_int32(), ctypes.c_int32()
        shape = (ctypes.c_int64 * MAX_RANK)()
        check(lib().zjai_checkpoint_info(self._h, name.encode(), ctypes.byref(dt),
                                         ctypes.byref(rank), shape))
        return dt.value, tuple(shape[:rank.value])

    def raw(self, name: str):
        """``Checkpoint::raw``: (dtype name, shape, contiguous little-endian bytes)."""
        dt, shape = self._dtype_shape(name)
        n = int(np.prod(shape, dtype=np.int64)) * DTYPES[dt][1].itemsize
        buf = ctypes.create_string_buffer(max(n, 1))
        check(lib().zjai_checkpoint_read(self._h, name.encode(), buf, n))
        return DTYPES[dt][0], shape, buf.raw[:n]

    def array(self, name: str) -> np.ndarray:
        """The tensor as a numpy array of its own dtype."""
        dt, shape = self._dtype_shape(name)
        _, _, b = self.raw(name)
        return np.frombuffer(b, DTYPES[dt][1]).reshape(shape).copy()

    def f32(self, name: str) -> np.ndarray:
        """``Checkpoint::f32``: an f32 tensor, or an f16 one upcast exactly."""
        _, shape = self._dtype_shape(name)
        out = np.empty(shape, np.float32)
        check(lib().zjai_checkpoint_read_f32(self._h, name.encode(),
                                             out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                             out.size))
        return out

    def ints(self) -> list[tuple[str, int]]:
        out = []
        for i in range(self._ni):
            v = ctypes.c_int64()
            nm = _name(lambda *a: lib().zjai_checkpoint_int_at(*a, ctypes.byref(v)), self._h, i)
            out.append((nm, v.value))
        return out

    def int(self, name: str):
        return dict(self.ints()).get(name)

    def lists(self) -> list[tuple[str, list[float]]]:
        out = []
        for i in range(self._nl):
            n = ctypes.c_size_t()
            buf = ctypes.create_string_buffer(1024)
            check(lib().zjai_checkpoint_list_at(self._h, i, buf, len(buf), None, 0, ctypes.byref(n)))
            vals = (ctypes.c_double * max(n.value, 1))()
            check(lib().zjai_checkpoint_list_at(self._h, i, buf, len(buf), vals, n.value,
                                                ctypes.byref(n)))
            out.append((buf.value.decode(), list(vals[:n.value])))
        return out

    def list(self, name: str):
        return dict(self.lists()).get(name)

    def write_zjm(self, names, f16: bool = False) -> bytes:
        """``write_zjm`` / ``write_zjm_f16`` (src/weights/packed.rs:166-225)."""
        c_names = (ctypes.c_char_p * max(len(names), 1))(*[n.encode() for n in names])
        size = ctypes.c_size_t()
        check(lib().zjai_checkpoint_write_zjm(self._h, c_names, len(names), int(f16), None, 0,
                                              ctypes.byref(size)))
        buf = ctypes.create_string_buffer(max(size.value, 1))
        check(lib().zjai_checkpoint_write_zjm(self._h, c_names, len(names), int(f16), buf,
                                              size.value, ctypes.byref(size)))
        return buf.raw[:size.value]

    def __del__(self):
        try:
            if self._h:
                lib().zjai_checkpoint_destroy(self._h)
                self._h = None
        except Exception:
            pass


class PackedBundle:
    """``PackedBundle`` (src/weights/packed.rs:290-384): files of ``ZJB1`` / ``ZJB2`` bundles by
    relative path; a path already present keeps its first copy."""

    def __init__(self, data: bytes):
        self._h = ctypes.c_void_p()
        check(lib().zjai_bundle_parse(data, len(data), ctypes.byref(self._h)))

    @classmethod
    def parse(cls, data: bytes) -> "PackedBundle":
        return cls(bytes(data))

    def add(self, data: bytes) -> None:
        check(lib().zjai_bundle_add(self._h, bytes(data), len(data)))

    def paths(self) -> list[str]:
        n = ctypes.c_int32()
        check(lib().zjai_bundle_count(self._h, ctypes.byref(n)))
        return [_name(lib().zjai_bundle_path, self._h, i) for i in range(n.value)]

    def contains(self, rel: str) -> bool:
        p, n = ctypes.c_void_p(), ctypes.c_size_t()
        return lib().zjai_bundle_get(self._h, rel.encode(), ctypes.byref(p), ctypes.byref(n)) == _lib.OK

    def read(self, rel: str) -> bytes:
        """``ModelSource::read``: a file's bytes."""
        p, n = ctypes.c_void_p(), ctypes.c_size_t()
        check(lib().zjai_bundle_get(self._h, rel.encode(), ctypes.byref(p), ctypes.byref(n)))
        return ctypes.string_at(p, n.value) if n.value else b""

    def checkpoint(self, rel: str) -> Checkpoint:
        return Checkpoint(self.read(rel))

    def notice(self) -> str:
        n = ctypes.c_size_t()
        check(lib().zjai_bundle_notice(self._h, None, 0, ctypes.byref(n)))
        buf = ctypes.create_string_buffer(n.value + 1)
        check(lib().zjai_bundle_notice(self._h, buf, len(buf), ctypes.byref(n)))
        return buf.raw[:n.value].decode()

    def __del__(self):
        try:
            if self._h:
                lib().zjai_bundle_destroy(self._h)
                self._h = None
        except Exception:
            pass


def write_bundle(files, notice: str, f16: bool = False) -> bytes:
    """``write_bundle`` / ``write_bundle_f16`` (src/weights/packed.rs:235-334): ``files`` is a
    list of (relative path, bytes)."""
    n = len(files)
    paths = (ctypes.c_char_p * max(n, 1))(*[p.encode() for p, _ in files])
    keep = [ctypes.create_string_buffer(bytes(b), max(len(b), 1)) for _, b in files]
    ptrs = (ctypes.c_void_p * max(n, 1))(*[ctypes.cast(k, ctypes.c_void_p) for k in keep])
    sizes = (ctypes.c_size_t * max(n, 1))(*[len(b) for _, b in files])
    size = ctypes.c_size_t()
    check(lib().zjai_bundle_write(paths, ptrs, sizes, n, notice.encode(), int(f16), None, 0,
                                  ctypes.byref(size)))
    buf = ctypes.create_string_buffer(max(size.value, 1))
    check(lib().zjai_bundle_write(paths, ptrs, sizes, n, notice.encode(), int(f16), buf, size.value,
                                  ctypes.byref(size)))
    return buf.raw[:size.value]
