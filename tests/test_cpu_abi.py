"""CPU checks of the C-ABI library: it loads, exports every symbol the header declares, and its host-only
entry points (sizes, validation) behave; no kernel is launched."""
import ctypes as C
import os
import re
import subprocess

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "quanta_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\**\s+\**(qh_[a-z0-9_]+)\s*\(", text, flags=re.M)


def test_header_declarations_are_exported(qh):
    names = declared_functions()
    assert len(names) >= 15
    assert tuple(names) == qh.EXPORTS
    out = subprocess.run(["nm", "-D", "--defined-only", qh.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r" T (qh_[a-z0-9_]+)$", out, flags=re.M))
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    lib = qh.lib()
    for n in names:
        assert hasattr(lib, n)


def test_sizes_follow_qnt_layout(qh):
    L = qh.lib()
    assert L.qh_quant_bytes(qh.Q8_0, 4864, 896) == 4864 * 896
    assert L.qh_quant_bytes(qh.Q4_0, 4864, 896) == 4864 * 896 // 2
    assert L.qh_quant_bytes(qh.F16, 3, 5) == 30 and L.qh_quant_bytes(qh.F32, 3, 5) == 60
    assert L.qh_tensor_bytes(qh.Q8_0, 4864, 896) == 4630528  # 1.0625 B per weight
    assert L.qh_tensor_bytes(qh.Q4_0, 4864, 896) == 2451456  # 0.5625 B per weight
    assert L.qh_tensor_bytes(qh.F16, 151936, 28) == 151936 * 28 * 2
    assert L.qh_shortlist_workspace_bytes(151936, 896, 1) > 151936
    assert L.qh_shortlist_workspace_bytes(151936, 896, 257) == 0  # above the top_k limit
    assert L.qh_shortlist_workspace_bytes(151936, 896, 256) > 0
    assert L.qh_shortlist_workspace_bytes(151936, 96, 1) == 0  # hidden size not a multiple of 64
    assert L.qh_shortlist_workspace_bytes(151936, 896, 0) == 0


@pytest.mark.parametrize("dtype,rows,cols,ptr,code", [
    (0, 4, 32, 256, 2),       # f32 is not a quantized dtype for matvec
    (2, 4, 48, 256, 3),       # cols % 32
    (2, 0, 32, 256, 3),       # empty
    (3, 4, 64, 260, 4),       # misaligned data
    (2, 4, 64, 0, 1),         # null data
])
def test_validation_codes(qh, dtype, rows, cols, ptr, code):
    L = qh.lib()
    W = qh.qh_tensor(dtype, rows, cols, ptr or None)
    assert L.qh_matvec_q(C.c_void_p(16), C.byref(W), C.c_void_p(16), C.c_void_p(16), 0, max(rows, 0), None) == code
    assert L.qh_last_error()


def test_range_and_pointer_checks(qh):
    L = qh.lib()
    W = qh.qh_tensor(qh.Q8_0, 64, 64, 4096)
    assert L.qh_matvec_q(C.c_void_p(16), C.byref(W), C.c_void_p(16), C.c_void_p(16), 10, 65, None) == 1
    assert L.qh_matvec_q(C.c_void_p(16), C.byref(W), C.c_void_p(16), C.c_void_p(16), 5, 4, None) == 1
    assert L.qh_matvec_q(None, C.byref(W), C.c_void_p(16), C.c_void_p(16), 0, 64, None) == 1
    assert L.qh_matvec_q(C.c_void_p(16), C.byref(W), C.c_void_p(24), C.c_void_p(16), 0, 64, None) == 4
    # empty ranges and empty batches are no-ops
    assert L.qh_matvec_q(C.c_void_p(16), C.byref(W), C.c_void_p(16), C.c_void_p(16), 3, 3, None) == 0
    assert L.qh_matmul_q(C.c_void_p(16), 64, C.byref(W), C.c_void_p(16), C.c_void_p(16), 0, 0, 64, None) == 0
    assert L.qh_matmul_q(C.c_void_p(16), 32, C.byref(W), C.c_void_p(16), C.c_void_p(16), 4, 0, 64, None) == 1
    assert L.qh_quantize_q8(C.c_void_p(16), 1, 40, C.c_void_p(16), C.c_void_p(16), None) == 3
    assert L.qh_argmax(C.c_void_p(16), 0, C.c_void_p(16), C.c_void_p(16), 4096, None) == 1
    need = L.qh_argmax_workspace_bytes(151936)
    assert 0 < need <= 8192 and L.qh_argmax_workspace_bytes(0) == 0
    assert L.qh_argmax(C.c_void_p(16), 151936, C.c_void_p(16), C.c_void_p(16), need - 1, None) == 6
    assert L.qh_argmax(C.c_void_p(16), 151936, C.c_void_p(16), None, need, None) == 6


def test_shortlist_argument_checks(qh):
    L = qh.lib()
    V, D = 1000, 64
    h8 = qh.qh_tensor(qh.Q8_0, V, D, 4096)
    h4 = qh.qh_tensor(qh.Q4_0, V, D, 8192)
    he = qh.qh_tensor(qh.F16, V, D // 32, 16384)
    bad = qh.qh_tensor(qh.F16, V, D // 32 + 1, 16384)
    out = qh.qh_head_out(16, 16, 16, 16, 16)
    q = qh.qh_head_query(1, 0, None, 0)
    ws = L.qh_shortlist_workspace_bytes(V, D, 1)
    call = lambda e, qq, w: L.qh_shortlist_head(C.byref(h8), C.byref(h4), C.byref(e), C.c_void_p(16),
                                                C.c_void_p(16), C.byref(qq), C.byref(out), C.c_void_p(4096), w, None)
    assert call(bad, q, ws) == 3                     # bound tensor shape (model.cpp:49-58)
    assert call(he, q, ws - 1) == 6                  # workspace too small
    assert call(he, qh.qh_head_query(0, 0, None, 0), ws) == 7
    assert call(he, qh.qh_head_query(257, 0, None, 0), ws) == 7
    assert call(he, qh.qh_head_query(1, 0, None, 3), ws) == 1  # must count without a list
    swapped = lambda: L.qh_shortlist_head(C.byref(h4), C.byref(h8), C.byref(he), C.c_void_p(16), C.c_void_p(16),
                                          C.byref(q), C.byref(out), C.c_void_p(4096), ws, None)
    assert swapped() == 2


def test_package_fails_loudly_without_library(qh, monkeypatch, tmp_path):
    monkeypatch.setattr(qh, "LIB_PATH", str(tmp_path / "missing.so"))
    monkeypatch.setattr(qh, "_lib", None)
    with pytest.raises(qh.QHError, match="no CPU fallback"):
        qh.lib()


def test_noalloc_entry_point_host_checks(qh):
    """The no-allocation shortlist entry point: its scratch size in the header and the binding agree, and bad
    arguments are refused on the host before any device work."""
    text = open(HEADER).read()
    m = re.search(r"#define QH_NOALLOC_SCRATCH_BYTES \(\(size_t\)(\d+) << (\d+)\)", text)
    assert m and int(m.group(1)) << int(m.group(2)) == qh.NOALLOC_SCRATCH_BYTES
    L = qh.lib()
    assert L.qh_shortlist_head_noalloc(None, None, None, None, None, None, None, None) == qh.ERR_ARG
    assert b"null argument" in L.qh_last_error()


def test_noalloc_refuses_oversized_head(qh):
    """A head whose workspace exceeds the scratch array: QH_ERR_NOMEM from the size check, which runs before the
    library touches a device (the descriptors point at no memory, so nothing may be launched)."""
    L = qh.lib()
    V, D = 1_000_000, 896  # supported (at most 1,048,576 rows), with a workspace beyond the scratch array
    assert L.qh_shortlist_workspace_bytes(V, D, 1) > qh.NOALLOC_SCRATCH_BYTES
    h8 = qh.qh_tensor(qh.Q8_0, V, D, 4096)
    h4 = qh.qh_tensor(qh.Q4_0, V, D, 8192)
    he = qh.qh_tensor(qh.F16, V, D // 32, 16384)
    out = qh.qh_head_out(16, 16, 16, 16, 16)
    q = qh.qh_head_query(1, 0, None, 0)
    rc = L.qh_shortlist_head_noalloc(C.byref(h8), C.byref(h4), C.byref(he), C.c_void_p(16), C.c_void_p(16),
                                     C.byref(q), C.byref(out), None)
    assert rc == qh.ERR_NOMEM and b"scratch array" in L.qh_last_error()


def test_forced_allocation_failure(qh):
    """qh_fault_alloc: the armed allocation fails with QH_ERR_NOMEM before any HIP call (so on a machine without a
    GPU too), the out pointer is cleared, and the hook disarms itself after firing."""
    L = qh.lib()
    p = C.c_void_p(1234)
    try:
        assert L.qh_fault_alloc(0) == 0
        assert L.qh_malloc(C.byref(p), 4096) == qh.ERR_NOMEM
        assert p.value is None
        assert b"forced allocation failure" in L.qh_last_error()
        assert L.qh_malloc(C.byref(p), 0) == 0  # an empty allocation is no allocation: nothing to fail
    finally:
        L.qh_fault_alloc(-1)


def _desc_and_tensors(qh, flags=0, kv_f32=0, ffn=512, lm=None, shortlist=True, emb=2):
    """A one-layer model descriptor and tensor list (descriptors at made-up, aligned addresses: only the host checks
    of qh_decoder_create may run on them)."""
    V, D, kvd, F = 1024, 256, 64, ffn
    desc = qh.qh_model_desc(V, D, 1, 4, 1, 64, F, 128, 0, 1e6, 1e-6, flags, kv_f32)
    addr = iter(range(1 << 20, 1 << 30, 1 << 16))
    t = lambda dt, r, c: qh.qh_tensor(dt, r, c, next(addr))
    none = qh.qh_tensor(0, 0, 0, None)
    ts = [t(emb, V, D), t(qh.F32, 1, D), t(qh.F32, 1, D), t(qh.Q4_0, D, D), t(qh.Q4_0, kvd, D),
          t(qh.Q4_0, kvd, D), t(qh.Q4_0, D, D), none, none, none, t(qh.F32, 1, D), t(qh.Q4_0, F, D),
          t(qh.Q4_0, F, D), t(qh.Q4_0, D, F)]
    ts += [t(qh.Q4_0, V, D), t(qh.F16, V, D // 32)] if shortlist else [none, none]
    if lm is not None:
        ts.append(t(*lm))
    return desc, (qh.qh_tensor * len(ts))(*ts), len(ts)


@pytest.mark.parametrize("case,code,msg", [
    (dict(flags=2), "ERR_ARG", b"unknown flags"),
    (dict(flags=1, ffn=480), "ERR_SHAPE", b"ffn_dim % 256"),  # as model.cpp:39-42
    (dict(kv_f32=2), "ERR_ARG", b"kv_f32"),
    (dict(lm=(7, 1024, 256)), "ERR_DTYPE", b"lm_head: dtype 7 is not"),
    (dict(lm=(1, 1024, 256)), "ERR_SHAPE", b"bad shortlist head tensors"),  # an F16 LM head with the shortlist
    (dict(lm=(2, 1000, 256)), "ERR_SHAPE", b"lm_head is 1000 x 256"),
    (dict(lm=(3, 1024, 256)), "ERR_SHAPE", b"bad shortlist head tensors"),  # Q8_0 with the shortlist (model.cpp:51)
    (dict(emb=3), "ERR_SHAPE", b"bad shortlist head tensors"),  # a tied Q4_0 LM head with the shortlist tensors
    (dict(emb=16), "ERR_ARG", b"nibble-plane LM head is its own shortlist"),
    (dict(lm=(16, 1024, 256)), "ERR_ARG", b"nibble-plane LM head is its own shortlist"),
    (dict(lm=(16, 1024, 96), shortlist=False), "ERR_SHAPE", b"lm_head: bad shape 1024 x 96"),
])
def test_decoder_create_option_checks(qh, case, code, msg):
    """qh_decoder_create's checks of the load-time options (flags, kv_f32, an untied lm_head.weight), refused on the
    host before any device work."""
    desc, ts, n = _desc_and_tensors(qh, **case)
    h = C.c_void_p()
    rc = qh.lib().qh_decoder_create(C.byref(desc), ts, n, C.byref(h))
    assert rc == getattr(qh, code) and msg in qh.lib().qh_last_error() and not h.value


def test_decoder_create_tensor_count(qh):
    desc, ts, n = _desc_and_tensors(qh, lm=(2, 1024, 256))
    h = C.c_void_p()
    assert qh.lib().qh_decoder_create(C.byref(desc), ts, n - 2, C.byref(h)) == qh.ERR_ARG
    assert b"needs 16 or 17" in qh.lib().qh_last_error()


def test_planes_entry_points_host_checks(qh):
    """The nibble-plane head: the layout's size equals the Q8_0 tensor's, and bad arguments are refused on the host
    (descriptors at made-up aligned addresses: nothing may be launched)."""
    L = qh.lib()
    V, D = 151936, 896
    assert L.qh_tensor_bytes(qh.Q8_0_PLANES, V, D) == L.qh_tensor_bytes(qh.Q8_0, V, D)
    assert L.qh_quant_bytes(qh.Q8_0_PLANES, V, D) == V * D
    h8 = qh.qh_tensor(qh.Q8_0, V, D, 1 << 30)
    assert L.qh_head_planes(C.byref(h8), C.c_void_p((1 << 30) + 4096), None) == qh.ERR_ARG  # overlapping
    assert b"overlap" in L.qh_last_error()
    assert L.qh_head_planes(C.byref(h8), C.c_void_p((1 << 33) + 8), None) == qh.ERR_ALIGN
    h4 = qh.qh_tensor(qh.Q4_0, V, D, 1 << 30)
    assert L.qh_head_planes(C.byref(h4), C.c_void_p(1 << 33), None) == qh.ERR_DTYPE
    odd = qh.qh_tensor(qh.Q8_0, V, 96, 1 << 30)
    assert L.qh_head_planes(C.byref(odd), C.c_void_p(1 << 33), None) == qh.ERR_SHAPE
    out = qh.qh_head_out(16, 16, 16, 16, 16)
    q = qh.qh_head_query(1, 0, None, 0)
    call = lambda t, ws_bytes: L.qh_shortlist_planes(C.byref(t), C.c_void_p(16), C.c_void_p(16), C.byref(q),
                                                     C.byref(out), C.c_void_p(4096), ws_bytes, None)
    assert call(h8, 1 << 30) == qh.ERR_DTYPE  # a plain Q8_0 descriptor is not the plane layout
    pl = qh.qh_tensor(qh.Q8_0_PLANES, V, D, 1 << 30)
    assert L.qh_validate_tensor(C.byref(pl)) == 0
    assert call(pl, 16) == qh.ERR_NOMEM  # workspace too small
    q.top_k = 0
    assert call(pl, 1 << 30) == qh.ERR_UNSUPPORTED


def test_prefill_stack_argument_checks(qh):
    """qh_decoder_set_prefill_stack refuses a null decoder and stacks that are no multiple of 32 in [32, 1024] before
    it touches the decoder (a made-up handle here)."""
    L = qh.lib()
    assert L.qh_decoder_set_prefill_stack(None, 64) == qh.ERR_ARG
    for bad in (0, 16, 48, 1056, -32):
        assert L.qh_decoder_set_prefill_stack(C.c_void_p(4096), bad) == qh.ERR_ARG
        assert b"multiple of 32" in L.qh_last_error()
