"""CPU: the Rust FFI block a maintainer would add binds exactly the
entry points include/zjai_hip.h declares -- same names, same parameter counts -- and its
constants carry the header's values, so the documented binding cannot drift from the C-ABI."""

import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header():
    src = open(os.path.join(ROOT, "include", "zjai_hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    fns = {}
    for name, args in re.findall(r"ZJAI_API\s+int32_t\s+(\w+)\s*\((.*?)\);", src, flags=re.S):
        fns[name] = 0 if not args.strip() else len(args.split(","))
    consts = {}
    for name, val in re.findall(r"#define\s+(ZJAI_[A-Z0-9_]+)\s+(.+)", src):
        v = re.sub(r"(?<=[0-9a-fA-F])u\b", "", val.strip())
        try:
            consts[name] = int(eval(v, {}, {}))
        except Exception:
            pass
    return fns, consts


def _rust():
    doc = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    block = doc[doc.index("## 1. The FFI block"):doc.index("## 2. The safe wrapper")]
    block = block[block.index("```rust"):]
    fns = {}
    for name, args in re.findall(r"pub fn (\w+)\((.*?)\)\s*->\s*i32;", block, flags=re.S):
        fns[name] = 0 if not args.strip() else len(args.split(","))
    consts = {n: int(eval(v.replace("_", ""), {}, {}))
              for n, v in re.findall(r"pub const (ZJAI_\w+): \w+ = ([^;]+);", block)}
    return fns, consts


def test_rust_block_binds_every_entry_point_with_its_parameter_count():
    hf, _ = _header()
    rf, _ = _rust()
    assert len(hf) >= 76
    assert set(rf) == set(hf), (sorted(set(hf) - set(rf)), sorted(set(rf) - set(hf)))
    for name, n in hf.items():
        assert rf[name] == n, (name, n, rf[name])


def test_rust_constants_carry_the_header_values():
    _, hc = _header()
    _, rc = _rust()
    assert len(rc) >= 40
    for name, v in rc.items():
        assert name in hc, name
        assert hc[name] == v, (name, hc[name], v)
