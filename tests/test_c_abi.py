"""CPU: a plain C99 program (tests/c/abi_host.c) that includes only include/zjai_hip.h calls the
host-side entry points -- tiling geometry, region grids, checkpoint and bundle readers, error
reporting -- through the C-ABI, built with gcc -std=c99 -pedantic under AddressSanitizer and
UndefinedBehaviorSanitizer (host code only: nothing here touches a device)."""

import os
import shutil
import subprocess

import pytest

from zenjpegai_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not installed")
def test_c99_consumer_under_sanitizers(tmp_path):
    _lib.lib()  # the library is built
    exe = tmp_path / "abi_host"
    libdir = os.path.dirname(_lib.LIB_PATH)
    cmd = ["gcc", "-std=c99", "-pedantic", "-Wall", "-Wextra", "-Werror", "-g", "-O1",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
           "-fno-omit-frame-pointer", "-I", os.path.join(ROOT, "include"),
           os.path.join(ROOT, "tests", "c", "abi_host.c"), "-o", str(exe),
           "-L", libdir, "-lzjai_hip", "-Wl,-rpath," + libdir]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=300)
    print(r.stdout, r.stderr[-4000:])
    assert r.returncode == 0, r.stderr[-4000:]
    assert "all checks passed" in r.stdout
