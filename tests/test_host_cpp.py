"""The C++ host side (fak_amd/host: compute.Backend, RocmBackend, the registry, the fused-MLP
and Q6_K seams) through its own C++ test program, tests/cpp/backend_test.cpp, which restates the
reference's backend tests (internal/compute/cuda_quant_test.go) against the oracle. Without a
device it runs the device-free cases and checks that no backend registers."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "cpp", "_build", "backend_test")


def _binary():
    if not os.path.exists(BIN):
        import importlib.util
        spec = importlib.util.spec_from_file_location("cpp_build", os.path.join(HERE, "cpp", "build.py"))
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build()
    return BIN


def _run(args, timeout):
    r = subprocess.run([_binary(), *args], capture_output=True, text=True, timeout=timeout)
    print(r.stdout, r.stderr, flush=True)
    return r


def test_host_cpp_device_free_cases():
    r = _run(["--cpu"], 120)
    assert r.returncode == 0, r.stdout
    for case in ("RegistrySemantics", "RegisterRocm", "HostTensorConstructors"):
        assert f"PASS {case}" in r.stdout


@pytest.mark.gpu
def test_host_cpp_backend_on_device():
    r = _run([], 120)
    assert r.returncode == 0, r.stdout
    for case in ("Q4KMatMulApproxMatchesRef", "Q4KBatchedMatMulApproxMatchesRef",
                 "Q8MatMulApproxMatchesRef", "Q8BatchedMatMulApproxMatchesRef", "QuantVRAMWitness",
                 "Q4KInt8RouteBitIdentical", "FusedMLPMatchesChain", "AsyncOutputsReadyAfterFence"):
        assert f"PASS {case}" in r.stdout
