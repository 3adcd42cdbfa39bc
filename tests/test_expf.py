"""The decoder's exp (quanta.cpp_amd/csrc/qh_math.h, glibc's expf method restated) over every binary32 input.

* host: tests/cpp/bin/expf_exhaustive compares the restatement with the host libm's expf on all 2^32 inputs. The
  variant the kernels use has no difference; the two other multiply-add associations each differ somewhere, so the
  check tells the associations apart.
* device (gpu): tests/cpp/bin/expf_device evaluates the same function on the MI355X for all 2^32 inputs and
  compares each with the host's result.
"""
import os
import re
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "cpp", "bin")


def _built(name):
    path = os.path.join(BIN, name)
    if not os.path.exists(path):
        subprocess.run(["make", "-s", "-C", os.path.join(HERE, "cpp"), f"bin/{name}"], check=True)
    return path


def test_host_expf_restatement_equals_libm_on_every_input():
    r = subprocess.run([_built("expf_exhaustive")], capture_output=True, text=True, timeout=600)
    counts = {int(v): int(n) for v, n in re.findall(r"expf variant (\d) \(fused=\d\): (\d+) of", r.stdout)}
    assert r.returncode == 0, r.stdout
    assert counts[2] == 0
    assert counts[0] > 0 and counts[1] > 0, "the other associations should differ somewhere"


@pytest.mark.gpu
def test_device_expf_equals_host_on_every_input(gpu):
    path = os.path.join(BIN, "expf_device")
    assert os.path.exists(path), "tests/cpp/bin/expf_device is not built (make -C tests/cpp)"
    r = subprocess.run([path], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 of 4294967296 inputs differ" in r.stdout
