"""GPU-free checks of the C ABI boundary (the pattern of the reference's
tools/cuda_abi_parity.py and build_cuda.sh strict header parse):

* the header is plain C (gcc -x c -fsyntax-only -std=c99 -Wall -Werror);
* libfakhip.so loads and exports every entry point include/fakhip.h declares;
* the ctypes declarations cover exactly the header's entry points;
* the library is built for gfx950 only.
No device compute is issued here.
"""
import os
import re
import subprocess

import pytest

from fak_amd import fakhip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fakhip.h")


def header_symbols():
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(fhip_\w+)\s*\(", txt)))


def test_header_is_plain_c():
    r = subprocess.run(["gcc", "-x", "c", "-std=c99", "-fsyntax-only", "-Wall", "-Wextra",
                        "-Werror", HEADER], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_library_exports_every_declared_symbol():
    lib = fakhip.load()
    syms = header_symbols()
    assert len(syms) >= 30
    missing = [s for s in syms if not hasattr(lib, s)]
    assert not missing, missing
    nm = subprocess.run(["nm", "-D", "--defined-only", fakhip.LIB_PATH], capture_output=True,
                        text=True, check=True).stdout
    exported = set(re.findall(r"\bT (fhip_\w+)", nm))
    assert set(syms) <= exported, sorted(set(syms) - exported)


def test_ctypes_declarations_match_header():
    assert sorted(fakhip.SIGNATURES) == header_symbols()


def test_packed_size_entries_are_pure_host_functions():
    """Size queries are host arithmetic: callable without a device."""
    lib = fakhip.load()
    assert lib.fhip_q4k_packed_bytes(18944, 3584) == 18944 * 14 * 144
    assert lib.fhip_q4k_packed_bytes(9, 512) == 16 * 2 * 144  # rows padded to 16
    assert lib.fhip_q4k_packed_bytes(9, 500) == 0            # invalid K
    assert lib.fhip_q8_0_packed_bytes(1536, 576) == 1536 * 18 * 34
    assert lib.fhip_q8_0_packed_bytes(16, 96) == 16 * 4 * 34  # 3 blocks padded to a pair


def test_built_for_gfx950_only():
    out = subprocess.run(["/opt/rocm/bin/roc-obj-ls", fakhip.LIB_PATH], capture_output=True,
                         text=True)
    if out.returncode != 0:
        pytest.skip("roc-obj-ls unavailable")
    targets = set(re.findall(r"gfx\w+", out.stdout))
    assert targets == {"gfx950"}, out.stdout


def test_init_without_device_fails_cleanly():
    """In a container with no GPU, fhip_init reports ENODEV rather than crashing."""
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU node is present")
    lib = fakhip.load()
    rc = lib.fhip_init(None, 0, None, None)
    assert rc != 0
    assert fakhip.last_error()
