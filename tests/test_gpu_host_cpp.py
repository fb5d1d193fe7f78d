"""Runs the C++ parity test of the reference-interface mirror
(ark_amd/host/ark_host.hpp, test source tests/cpp/test_host.cpp): Optimizer,
lr_now, step_all, record_overflow, restaurar_momentos and CheckpointV3
through the C ABI, every step checked bit for bit against the CPU oracle."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "_build", "test_host")


def test_cpp_mirror_matches_oracle():
    assert os.path.exists(BIN), f"{BIN} is not built: run __graft_entry__.build()"
    r = subprocess.run([BIN], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                       timeout=120)
    print(r.stdout[-4000:])
    assert r.returncode == 0 and "ark_host_test: OK" in r.stdout, r.stdout[-4000:]
