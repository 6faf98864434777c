"""Runs the C++ host-layer tests (tests/cpp/host_tests.cpp): orchestrator, registry, LINQ provider
and fusion planner, MatrixOperations and SparseOps. --cpu cases need no device; --gpu cases run
the kernels on gfx950 and compare with the CPU oracle."""
import os
import subprocess

import pytest

BIN = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "dotcompute_amd", "lib", "dc_host_tests")


def _run(flag: str, timeout: int) -> None:
    assert os.path.exists(BIN), "host tests not built: python -m dotcompute_amd.build"
    r = subprocess.run([BIN, flag], capture_output=True, text=True, timeout=timeout)
    print(r.stdout[-4000:])
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-2000:]


def test_host_layer_cpu():
    _run("--cpu", 300)


@pytest.mark.gpu
def test_host_layer_gpu():
    _run("--gpu", 600)
