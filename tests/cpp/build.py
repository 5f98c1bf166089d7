"""Build recipe for the C++ host-side test (test infrastructure): tests/cpp/backend_test.cpp ->
tests/cpp/_build/backend_test, linked against fak_amd/libfakhost.so + libfakhip.so and the
oracle (oracle/_build/liboracle.so), found at run time relative to the binary."""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
OUT = os.path.join(HERE, "_build", "backend_test")


def build(verbose: bool = False) -> str:
    os.makedirs(os.path.dirname(OUT), exist_ok=True)
    tmp = OUT + ".tmp%d" % os.getpid()
    cmd = ["g++", "-std=c++17", "-O2", "-Wall", "-Wextra", os.path.join(HERE, "backend_test.cpp"),
           "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROOT, "fak_amd", "host"),
           "-I", os.path.join(ROOT, "oracle"),
           "-L", os.path.join(ROOT, "fak_amd"), "-lfakhost", "-lfakhip",
           "-L", os.path.join(ROOT, "oracle", "_build"), "-loracle", "-lpthread",
           "-Wl,-rpath,$ORIGIN/../../../fak_amd:$ORIGIN/../../../oracle/_build", "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"g++ failed for backend_test:\n{r.stdout}{r.stderr}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
