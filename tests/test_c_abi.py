"""The C ABI from C: tests/c_abi/abi_smoke.c, compiled with gcc as C99 against
include/paroquant_hip.h and linked to the built library, makes host-side calls
only (version, workspace rules, argument checks, empty inputs), so it runs
without a GPU."""

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIBDIR = os.path.join(ROOT, "alpamayo_amd")


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_c_caller(tmp_path):
    if not os.path.exists(os.path.join(LIBDIR, "libparoquant_hip.so")):
        pytest.fail("libparoquant_hip.so is not built")
    exe = str(tmp_path / "abi_smoke")
    cc = ["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"),
          os.path.join(ROOT, "tests", "c_abi", "abi_smoke.c"), "-L", LIBDIR, "-lparoquant_hip",
          f"-Wl,-rpath,{LIBDIR}", "-o", exe]
    r = subprocess.run(cc, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "ok (0 failures)" in r.stdout
