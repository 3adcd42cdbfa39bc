"""Runs the C++ self-test of the drop-in surface (tests/cpp/selftest.cpp) on the GPU."""
import os
import subprocess

import pytest

from conftest import ROOT

pytestmark = pytest.mark.gpu

BIN = os.path.join(ROOT, "tests", "cpp", "bin", "selftest")


def test_cpp_selftest_all_pass(gpu):
    assert os.path.exists(BIN), "tests/cpp/bin/selftest is not built (make -C tests/cpp)"
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "selftest: ALL PASS" in r.stdout
    assert r.stdout.count("PASS") >= 9
