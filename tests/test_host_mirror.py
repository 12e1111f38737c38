"""Runs the C++ host-side tests (tests/cpp/test_host_mirror.cpp): the reference's operator interface
mirrored in C++ above the C-ABI. CPU mode checks error mapping, table flattening and the no-GPU
path; GPU mode checks the HIP kernel behind ComputePagedAttention against the CPU oracle."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
BIN = os.path.join(HERE, "cpp", "test_host_mirror")


def _run(mode, timeout):
    r = subprocess.run([BIN, mode], capture_output=True, text=True, timeout=timeout)
    print(r.stdout)
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-2000:]
    assert " 0 failed" in r.stdout


def test_host_mirror_cpu():
    # built here when absent (plain g++; the HIP library itself must already be built)
    subprocess.run(["make", "-s", "-C", os.path.join(HERE, "cpp")], check=True)
    _run("--cpu", 120)


@pytest.mark.gpu
def test_host_mirror_gpu():
    assert os.path.exists(BIN), "tests/cpp/test_host_mirror is not built: run __graft_entry__.build()"
    _run("--gpu", 300)
