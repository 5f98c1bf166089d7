"""Build libfakhip.so (the gfx950 HIP backend) in-tree with hipcc.

Every .hip file under fak_amd/csrc is compiled for gfx950 only and linked into
fak_amd/libfakhip.so. Objects go to fak_amd/_build/. Packed-FP32 instruction selection is
disabled (`-Xclang -target-feature -Xclang -packed-fp32-ops`); hipcc's host pass warns that it
does not know the feature, which is harmless.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libfakhip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
CXXFLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
    "-Wall", "-Wno-unused-result",
]


# Files whose results must be bit-identical to the reference's Go arithmetic, which never fuses
# multiply-add on amd64: hipcc contracts a*b+c into fma by default (pragmas included), so these
# are compiled with contraction off.
NO_CONTRACT = {"q8_hal.hip", "q4k_layout.hip", "q4k_i8route.hip", "q6k.hip"}

RESOURCE_REMARK = "kernel-resource-usage"


# Kernels allowed a small, measured spill (mangled-name fragment -> bytes per lane): the
# three-workgroups-per-CU prefill GEMM keeps one 16-byte staging value in scratch once per
# super-block (measured faster than the spill-free two-workgroup form: 116 vs 131 us at M=512).
SCRATCH_ALLOWED = {"quant_gemm32_kernelILi0ELi1ELi3E": 32}


def scratch_kernels(remarks: str) -> list[tuple[str, int]]:
    """(kernel, bytes/lane) for every kernel whose resource-usage remark reports scratch."""
    out, name = [], None
    for line in remarks.splitlines():
        if "Function Name:" in line:
            name = line.split("Function Name:")[1].split("[")[0].strip()
        elif "ScratchSize [bytes/lane]:" in line and name:
            n = int(line.split("ScratchSize [bytes/lane]:")[1].split("[")[0])
            if n:
                out.append((name, n))
    return out


def _compile(src: str, verbose: bool) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    extra = ["-ffp-contract=off"] if os.path.basename(src) in NO_CONTRACT else []
    cmd = [HIPCC, *CXXFLAGS, *extra, f"-Rpass-analysis={RESOURCE_REMARK}", "-c", src, "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = r.stdout + r.stderr
    msgs = "\n".join(l for l in out.splitlines()
                     if "packed-fp32-ops" not in l and RESOURCE_REMARK not in l and l.strip())
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{msgs}")
    if msgs and verbose:
        print(msgs, flush=True)
    # Register spills to scratch memory cost these bandwidth-bound kernels far more than they
    # save; every kernel must fit its registers, except the few listed in SCRATCH_ALLOWED.
    spills = [(k, n) for k, n in scratch_kernels(out)
              if not any(pat in k and n <= cap for pat, cap in SCRATCH_ALLOWED.items())]
    if spills:
        raise RuntimeError(f"{src}: kernels use scratch memory (register spills): {spills}")
    return obj


HOST = os.path.join(HERE, "host")
HOST_LIB = os.path.join(HERE, "libfakhost.so")
HOST_CXXFLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-I", os.path.join(ROOT, "include")]


def build_host(verbose: bool = False) -> str:
    """The C++ host side (fak_amd/host: the compute.Backend seam over the C ABI) ->
    fak_amd/libfakhost.so, linked against libfakhip.so (found next to it at run time)."""
    srcs = sorted(glob.glob(os.path.join(HOST, "*.cpp")))
    tmp = HOST_LIB + ".tmp%d" % os.getpid()
    cmd = ["g++", *HOST_CXXFLAGS, "-shared", *srcs, "-L", HERE, "-lfakhip",
           "-Wl,-rpath,$ORIGIN", "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"g++ failed for the host library:\n{r.stdout}{r.stderr}")
    os.replace(tmp, HOST_LIB)
    return HOST_LIB


def build(verbose: bool = False, jobs: int = 8) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    with cf.ThreadPoolExecutor(max_workers=min(jobs, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), srcs))
    tmp = LIB + ".tmp%d" % os.getpid()
    cmd = [HIPCC, "-shared", f"--offload-arch={ARCH}", "-fPIC", *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    build_host(verbose)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
