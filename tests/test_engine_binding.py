"""CPU checks of the reference-side binding (no kernel runs).

- quanta_ops.h compiles on its own (standalone types) and, with QUANTA_HIP_ENGINE, together with the reference
  engine's own headers and sources that call the kernels (ops.h, model.h, checks.cpp, model.cpp): the types come from
  the engine, so nothing is defined twice;
- oracle/_ref/quanta_hip, the reference engine and CLI built by `make -C oracle engine` with ops_dispatch.cpp replaced
  by ops_hip.cpp, takes matvec_q / matmul_q / shortlist_head from the HIP library: its Model::shortlist_head calls
  quanta::shortlist_head, and the C-ABI entry points it needs are left to libquanta_hip.so.
The checks that need the reference tree skip where it is not mounted.
"""
import os
import re
import subprocess

import pytest

from conftest import ROOT

REF = "/root/reference"
HOST = os.path.join(ROOT, "quanta.cpp_amd", "host")
INC = os.path.join(ROOT, "include")
ENGINE = os.path.join(ROOT, "oracle", "_ref", "quanta_hip")
CLANG = "/opt/rocm/llvm/bin/clang++"

needs_ref = pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "engine", "src")), reason="reference not mounted")


def syntax_check(src, *flags, stdin=None):
    cmd = [CLANG, "-std=c++17", "-fsyntax-only", *flags, src]
    r = subprocess.run(cmd, capture_output=True, text=True, input=stdin)
    assert r.returncode == 0, r.stderr[-3000:]


def test_standalone_header_compiles():
    syntax_check("-", "-x", "c++", f"-I{HOST}", stdin='#include "quanta_ops.h"\nint main() { return 0; }\n')


@needs_ref
def test_engine_mode_header_with_reference_sources():
    flags = ["-DQUANTA_HIP_ENGINE=1", "-DQUANTA_HIP=1", f"-I{REF}/engine/src", f"-I{HOST}", f"-I{INC}"]
    both = '#include "ops.h"\n#include "model.h"\n#include "quanta_ops.h"\n#include "checks.h"\n'
    syntax_check("-", "-x", "c++", *flags, stdin=both)
    for src in ("engine/src/checks.cpp", "engine/src/model.cpp"):
        syntax_check(os.path.join(REF, src), *flags, "-include", os.path.join(HOST, "quanta_ops.h"))
    syntax_check(os.path.join(HOST, "ops_hip.cpp"), *flags)


@needs_ref
def test_engine_binary_binds_the_hip_library():
    if not os.path.exists(ENGINE):
        pytest.skip("oracle/_ref/quanta_hip is not built (make -C oracle engine)")
    nm = subprocess.run(["nm", "-C", ENGINE], capture_output=True, text=True, check=True).stdout
    defined = set(re.findall(r"^[0-9a-f]+ T (.+)$", nm, flags=re.M))
    undefined = set(re.findall(r"^\s+U (\S+)$", nm, flags=re.M))
    for fn in ("quanta::matvec_q(", "quanta::matmul_q(", "quanta::shortlist_head(", "quanta::matvec_q_ref("):
        assert any(d.startswith(fn) for d in defined), fn
    assert {"qh_matvec_q", "qh_matmul_q", "qh_shortlist_head"} <= undefined
    dis = subprocess.run(["objdump", "-d", "--no-show-raw-insn", "-C", ENGINE], capture_output=True, text=True,
                         check=True).stdout
    body = dis.split("<quanta::Model::shortlist_head(quanta::HeadQuery const&)>:", 1)[1].split("\n\n", 1)[0]
    assert "call" in body and "<quanta::shortlist_head(" in body
