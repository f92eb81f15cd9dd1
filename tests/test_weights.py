"""Weight readers (host only, no GPU): `.pth` checkpoints written by torch.save itself and the
packed ZJM1 / ZJB1 / ZJB2 containers (src/weights/{mod,zip,pickle,packed}.rs), checked against
the tensors that were saved, against `oracle.packed` (the documented layout, pinned below by a
hand-assembled file) and against the reference's own bundle tests (tests/packed_bundle.rs)."""

import io
import os
import struct
import tempfile
import zipfile

import numpy as np
import pytest
import torch

from oracle import packed as op
from zenjpegai_amd import _lib, synth
from zenjpegai_amd.weights import Checkpoint, PackedBundle, write_bundle


def _pth(sd, **kw) -> bytes:
    b = io.BytesIO()
    torch.save(sd, b, **kw)
    return b.getvalue()


def _model_error(fn, *a):
    with pytest.raises(_lib.HipError) as e:
        fn(*a)
    assert e.value.code == _lib.E_MODEL, e.value
    return str(e.value)


def _mixed_state_dict():
    g = torch.Generator().manual_seed(5)
    base = torch.randn(6, 8, generator=g)
    sd = {
        "conv.weight": torch.randn(4, 3, 3, 3, generator=g),
        "conv.bias": torch.randn(4, generator=g),
        "f64": torch.randn(3, 2, generator=g, dtype=torch.float64),
        "f16": torch.randn(7, generator=g).half(),
        "i64": torch.arange(-5, 7, dtype=torch.int64).reshape(3, 4),
        "i32": torch.arange(-3, 3, dtype=torch.int32),
        "i16": torch.tensor([-32768, 0, 32767], dtype=torch.int16),
        "i8": torch.tensor([[-128, 5], [127, -1]], dtype=torch.int8),
        "u8": torch.tensor([0, 200, 255], dtype=torch.uint8),
        "flag": torch.tensor([True, False, True]),
        "scalar": torch.tensor(2.5),
        "empty": torch.zeros(0, 4),
        # views of one storage: offsets, a transpose and a strided slice
        "view.t": base.t(),
        "view.rows": base[2:5],
        "view.step": base[::2, 1::3],
        "param": torch.nn.Parameter(torch.randn(2, 2, generator=g)),
        "epoch": 12,
        "neg": -3,
    }
    return sd


def _check_tensors(ck, sd):
    for name, v in sd.items():
        if not isinstance(v, torch.Tensor):
            continue
        want = v.detach().contiguous().numpy()
        got = ck.array(name)
        assert got.shape == want.shape, name
        assert got.dtype == want.dtype, name
        assert np.array_equal(got, want), name


@pytest.mark.parametrize("protocol", [2, 3, 4, 5])
def test_pth_written_by_torch_save_reads_back_exactly(protocol):
    sd = _mixed_state_dict()
    ck = Checkpoint.parse(_pth(sd, pickle_protocol=protocol))
    assert not ck.packed
    tensors = [k for k, v in sd.items() if isinstance(v, torch.Tensor)]
    assert ck.tensor_names() == tensors  # file order
    assert ck.ints() == [("epoch", 12), ("neg", -3)]
    assert ck.int("epoch") == 12 and ck.int("missing") is None
    _check_tensors(ck, sd)
    assert ck.info("conv.weight") == ("F32", (4, 3, 3, 3))
    assert ck.info("scalar") == ("F32", ())
    assert ck.info("absent") is None
    # f32() upcasts f16 exactly and refuses other dtypes
    assert np.array_equal(ck.f32("f16"), sd["f16"].float().numpy())
    _model_error(ck.f32, "i64")
    _model_error(ck.f32, "absent")


def test_module_state_dict_and_nested_dicts():
    """A real nn.Module state dict (OrderedDict with _metadata) inside a training-style
    checkpoint: nested dict leaves flatten to dotted names, numeric lists are kept, three
    levels deep at most (src/weights/mod.rs:78-126)."""
    m = torch.nn.Sequential(torch.nn.Conv2d(3, 4, 3), torch.nn.ReLU(), torch.nn.Conv2d(4, 2, 1))
    clip = {"E1B": {"MinList": [0.5, -1, 2.25], "MaxList": [1, 2], "Mixed": [1, "a"]}}
    deep = {"a": {"b": {"c": {"d": torch.ones(1)}}, "t": torch.ones(2)}}
    ck = Checkpoint.parse(_pth({"state_dict": m.state_dict(), "clip_thres": clip, "deep": deep,
                                "epoch": 3}))
    names = ck.tensor_names()
    for k, v in m.state_dict().items():
        assert np.array_equal(ck.array(f"state_dict.{k}"), v.numpy())
    assert "deep.a.t" in names and not any(n.startswith("deep.a.b.c") for n in names)
    assert ck.list("clip_thres.E1B.MinList") == [0.5, -1.0, 2.25]
    assert ck.list("clip_thres.E1B.MaxList") == [1.0, 2.0]
    assert ck.list("clip_thres.E1B.Mixed") is None
    assert ck.ints() == [("epoch", 3)]


def test_bfloat16_storage_is_rejected_as_the_reference_does():
    msg = _model_error(Checkpoint.parse, _pth({"w": torch.ones(2, dtype=torch.bfloat16)}))
    assert "BFloat16Storage" in msg


def _rezip(data: bytes, compression=zipfile.ZIP_STORED, drop=None) -> bytes:
    src = zipfile.ZipFile(io.BytesIO(data))
    out = io.BytesIO()
    with zipfile.ZipFile(out, "w", compression) as z:
        for info in src.infolist():
            if drop and info.filename.endswith(drop):
                continue
            z.writestr(info.filename, src.read(info.filename))
    return out.getvalue()


def test_zip64_archives_read_back(monkeypatch):
    """Python's zipfile, told that 16 bytes is the 32-bit limit, writes ZIP64 extra fields with
    saturated sizes / offsets for every member and a ZIP64 end record."""
    sd = _mixed_state_dict()
    monkeypatch.setattr(zipfile, "ZIP64_LIMIT", 16)
    z64 = _rezip(_pth(sd))
    monkeypatch.undo()
    assert struct.pack("<I", 0x06064B50) in z64 and struct.pack("<I", 0x07064B50) in z64
    ck = Checkpoint.parse(z64)
    _check_tensors(ck, sd)


def test_malformed_pth_files_are_model_errors():
    good = _pth({"w": torch.ones(3)})
    _model_error(Checkpoint.parse, _rezip(good, zipfile.ZIP_DEFLATED))
    _model_error(Checkpoint.parse, _rezip(good, drop="data.pkl"))
    _model_error(Checkpoint.parse, good[:-30])
    _model_error(Checkpoint.parse, b"\0" * 100)
    _model_error(Checkpoint.parse, b"")
    # a storage member missing: parsing succeeds, reading the tensor fails
    ck = Checkpoint.parse(_rezip(good, drop="data/0"))
    _model_error(ck.f32, "w")
    # the legacy (pre-zip) torch.save format is not a ZIP
    _model_error(Checkpoint.parse, _pth({"w": torch.ones(3)}, _use_new_zipfile_serialization=False))


def test_pickle_globals_are_never_called():
    """A data.pkl whose state dict holds `posix.system(...)`: the interpreter records the name
    and builds an opaque value; nothing runs and the tensor-free dict parses."""
    marker = os.path.join(tempfile.mkdtemp(), "ran")
    cmd = f"touch '{marker}'".encode()
    pkl = (b"\x80\x02}q\x00(X\x01\x00\x00\x00x" + b"cposix\nsystem\n"
           + b"X" + struct.pack("<I", len(cmd)) + cmd + b"\x85Rq\x01"
           + b"X\x05\x00\x00\x00epochK\x07u.")
    out = io.BytesIO()
    with zipfile.ZipFile(out, "w") as z:
        z.writestr("archive/data.pkl", pkl)
    ck = Checkpoint.parse(out.getvalue())
    assert not os.path.exists(marker)
    assert ck.tensor_names() == [] and ck.ints() == [("epoch", 7)]


def test_deeply_nested_and_cyclic_pickles_parse_without_recursion():
    """Values live in an arena: a list nested 400k deep (MARK x n, LIST x n) and a list that
    contains itself (via the memo) neither overflow the stack nor leak when released."""
    n = 400_000
    nested = b"\x80\x02}q\x00X\x01\x00\x00\x00a" + b"(" * n + b"l" * n + b"sX\x05\x00\x00\x00epochK\x03s."
    cyclic = b"\x80\x02}q\x00X\x01\x00\x00\x00b]q\x01h\x01as."
    for pkl in (nested, cyclic):
        out = io.BytesIO()
        with zipfile.ZipFile(out, "w") as z:
            z.writestr("a/data.pkl", pkl)
        ck = Checkpoint.parse(out.getvalue())
        assert ck.tensor_names() == []
    assert ck.ints() == []


def test_pickle_rejects_unknown_opcodes_and_truncation():
    for pkl in (b"\x80\x02}q\x00Z.", b"\x80\x02}q\x00(X\xff\xff\xff\x7f", b"\x80\x02(t", b"\x80\x09}."):
        out = io.BytesIO()
        with zipfile.ZipFile(out, "w") as z:
            z.writestr("a/data.pkl", pkl)
        _model_error(Checkpoint.parse, out.getvalue())


# --------------------------------------------------------------------------- packed files

# One f32 tensor "w" = [1, -2] and one integer entry "e" = 5, assembled by hand from the layout
# of src/weights/packed.rs:12-21: table = 16 + (2 + 1 + 2 + 8 + 16) + (2 + 1 + 8) = 56 bytes,
# padded to 64; payload 8 bytes at offset 64, padded to 128.
KNOWN_ZJM1 = bytes.fromhex(
    "5a4a4d31" "01000000" "01000000" "01000000"      # magic, version, 1 tensor, 1 int
    "0100" "77" "01" "01" "0200000000000000"          # "w", F32, rank 1, dim 2
    "4000000000000000" "0800000000000000"             # offset 64, 8 bytes
    "0100" "65" "0500000000000000"                    # "e" = 5
    + "00" * 8                                        # pad the 56-byte table to 64
    + "0000803f" "000000c0" + "00" * 56)              # 1.0, -2.0, pad to 128


def test_known_answer_zjm1_file():
    assert len(KNOWN_ZJM1) == 128
    tensors, ints = op.read_zjm(KNOWN_ZJM1)
    assert ints == [("e", 5)] and tensors["w"][0] == "F32"
    assert np.array_equal(tensors["w"][1], [1.0, -2.0])
    assert op.write_zjm([("w", "F32", np.array([1.0, -2.0], np.float32))], [("e", 5)]) == KNOWN_ZJM1
    ck = Checkpoint.parse(KNOWN_ZJM1)
    assert ck.packed and ck.tensor_names() == ["w"] and ck.ints() == [("e", 5)]
    assert np.array_equal(ck.f32("w"), [1.0, -2.0])
    assert ck.write_zjm(["w"]) == KNOWN_ZJM1  # the writer reproduces the file


def _layout_ok(data: bytes):
    """Offsets and lengths of a ZJM1 file: every payload 64-aligned inside the file, the file a
    multiple of 64."""
    tensors, _ = op.read_zjm(data)
    assert len(data) % 64 == 0
    return tensors


@pytest.mark.parametrize("f16", [False, True])
def test_zjm1_writer_matches_the_documented_layout(f16):
    sd = _mixed_state_dict()
    ck = Checkpoint.parse(_pth(sd))
    names = ck.tensor_names()
    got = ck.write_zjm(names, f16=f16)
    want = op.write_zjm([(n, ck.info(n)[0], ck.array(n)) for n in names], ck.ints(), f16=f16)
    assert got == want
    tensors = _layout_ok(got)
    back = Checkpoint.parse(got)
    assert back.packed and back.tensor_names() == names and back.ints() == ck.ints()
    for n in names:
        dt, arr = tensors[n]
        if f16 and ck.info(n)[0] == "F32":
            assert dt == "F16" and back.info(n)[0] == "F16"
            assert np.array_equal(back.f32(n), ck.array(n).astype(np.float16).astype(np.float32))
        else:
            assert np.array_equal(back.array(n), ck.array(n)), n
    # the packed file repacks to itself
    assert back.write_zjm(names, f16=f16) == got


def test_f16_packing_rounds_to_nearest_even_and_keeps_vr_vec_and_integers():
    """`write_zjm_f16` (src/weights/packed.rs:236-250) with the reference's f16 rule: ties to
    even, subnormals, overflow to infinity, signed zero, NaN; integers and `vr_vec.c` exact."""
    edge = np.array([0.0, -0.0, 1.0, 65504.0, 65520.0, 1e6, -1e6, 6.1e-5, 5.96e-8, 2.98e-8, 1e-9,
                     1.0009765625, 1.00048828125, 1.00146484375, np.inf, -np.inf, 0.1, -3.3],
                    np.float32)
    rnd = synth.normal(3, "f16pack", (4096,), 10.0).astype(np.float32)
    vals = np.concatenate([edge, rnd])
    sd = {"w": torch.from_numpy(vals), "vr_vec.c": torch.from_numpy(rnd[:16].copy()),
          "q": torch.arange(-4, 4, dtype=torch.int8), "epoch": 1}
    ck = Checkpoint.parse(_pth(sd))
    half = Checkpoint.parse(ck.write_zjm(ck.tensor_names(), f16=True))
    with np.errstate(over="ignore"):  # 1e6 and 65520 overflow to infinity, as they should
        want = vals.astype(np.float16)
    assert half.info("w")[0] == "F16" and half.info("vr_vec.c")[0] == "F32"
    assert np.array_equal(half.array("w"), want)
    assert np.array_equal(np.signbit(half.array("w")), np.signbit(want))
    assert np.array_equal(half.f32("w"), want.astype(np.float32))
    assert np.array_equal(half.array("vr_vec.c"), rnd[:16])
    assert np.array_equal(half.array("q"), sd["q"].numpy())
    assert half.ints() == [("epoch", 1)]
    nan = Checkpoint.parse(Checkpoint.parse(_pth({"n": torch.tensor([float("nan")])}))
                           .write_zjm(["n"], f16=True))
    assert np.isnan(nan.f32("n")).all()


def test_damaged_zjm1_files_are_rejected():
    good = bytearray(KNOWN_ZJM1)
    bad = []
    bad.append(bytes(good[:70]))                        # payload (64..72) cut off
    bad.append(b"ZJM2" + bytes(good[4:]))               # magic
    v = bytearray(good); v[4] = 2; bad.append(bytes(v))  # version
    d = bytearray(good); d[18 + 1] = 9; bad.append(bytes(d))  # dtype code 9
    r = bytearray(good); r[18 + 2] = 9; bad.append(bytes(r))  # rank 9 (and a table too short)
    o = bytearray(good); o[29] = 0x41; bad.append(bytes(o))   # offset 65, not 64-aligned
    ln = bytearray(good); ln[37] = 0x0c; bad.append(bytes(ln))  # 12 bytes for 2 x f32
    n = bytearray(good); n[8] = 0xff; n[9] = 0xff; n[10] = 0x7f; bad.append(bytes(n))  # count
    for i, b in enumerate(bad):
        with pytest.raises(_lib.HipError) as e:
            Checkpoint.parse(b)
        assert e.value.code in (_lib.E_MODEL, _lib.E_LIMIT), i


def _bundle_files():
    a = Checkpoint.parse(_pth(_mixed_state_dict()))
    b = Checkpoint.parse(_pth({"hyper_decoder.conv1.weight": torch.randn(4, 4, 3, 3), "epoch": 2}))
    return [("VM_common_int/Y_0.012.pth", a.write_zjm(a.tensor_names())),
            ("VM_common_int/common.pth", b.write_zjm(b.tensor_names())),
            ("notes.txt", b"any bytes work"),
            ("empty", b"")]


def test_bundle_round_trip_and_fixed_point():
    """tests/packed_bundle.rs:31-83: paths, notice, member bytes; rewriting a parsed bundle
    gives the same bytes; the writer matches the documented layout."""
    files = _bundle_files()
    data = write_bundle(files, "notice text")
    assert data == op.write_bundle(files, "notice text")
    assert len(data) % 64 == 0
    b = PackedBundle.parse(data)
    assert sorted(b.paths()) == sorted(p for p, _ in files)
    assert b.notice() == "notice text"
    for p, want in files:
        assert b.contains(p) and b.read(p) == want
    assert not b.contains("nope")
    _model_error(b.read, "nope")
    again = write_bundle([(p, b.read(p)) for p, _ in files], b.notice())
    assert again == data
    ck = b.checkpoint("VM_common_int/common.pth")
    assert ck.packed and ck.int("epoch") == 2


def test_bundles_merge_keeping_the_first_copy():
    files = _bundle_files()
    first = PackedBundle.parse(write_bundle(files[:2], "first"))
    first.add(write_bundle([(files[1][0], b"other"), files[2]], "second"))
    assert first.notice() == "first"
    assert first.read(files[1][0]) == files[1][1]  # first copy kept
    assert first.read(files[2][0]) == files[2][1]
    assert len(first.paths()) == 4


def test_zjb2_marks_f16_bundles():
    files = _bundle_files()[:2]
    half = [(p, Checkpoint.parse(d).write_zjm(Checkpoint.parse(d).tensor_names(), f16=True))
            for p, d in files]
    data = write_bundle(half, "n", f16=True)
    assert data[:4] == b"ZJB2" and data == op.write_bundle(half, "n", f16=True)
    b = PackedBundle.parse(data)
    ck = b.checkpoint(files[0][0])
    assert ck.info("conv.weight")[0] == "F16" and ck.info("i64")[0] == "I64"


def test_damaged_bundles_are_rejected():
    """tests/packed_bundle.rs:86-98."""
    data = write_bundle(_bundle_files(), "notice text")
    for bad in (data[:-100], data[:40], b"ZJB3" + data[4:], b"ZJB1", b"ZJB2", b"",
                data[:4] + struct.pack("<I", 2) + data[8:]):
        with pytest.raises(_lib.HipError) as e:
            PackedBundle.parse(bad)
        assert e.value.code in (_lib.E_MODEL, _lib.E_LIMIT)
    msg = _lib.last_error(None)
    assert msg


def test_a_synthesis_checkpoint_offers_every_weight_by_name():
    """The names the synthesis loaders look up (fuzz/fuzz_targets/common.rs:260-345) survive a
    torch.save -> ZJM1 -> ZJB1 trip bit for bit (what zjai_net_create_from_checkpoint reads)."""
    p = synth.random_params("hop", "y", seed=9)
    sd = {k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in p.items()}
    ck = Checkpoint.parse(_pth(sd))
    packed = Checkpoint.parse(ck.write_zjm(ck.tensor_names()))
    b = PackedBundle.parse(write_bundle([("m/y.pth", packed.write_zjm(packed.tensor_names()))], ""))
    final = b.checkpoint("m/y.pth")
    assert final.tensor_names() == list(p)
    for k, v in p.items():
        assert np.array_equal(final.f32(k), v), k
