"""GPU parity of the decode path: activation quantization, Q8_0 / Q4_0 GEMV, argmax.

Every check calls the C-ABI (through the ctypes binding) and compares with the oracle on the same seeded
inputs, bit for bit (integer block dots and the serial f32 chain must both match).
"""
import numpy as np
import pytest

from conftest import bits

pytestmark = pytest.mark.gpu

# Decode GEMV shapes of the benchmark workloads: Qwen2.5-0.5B q/o, k/v, gate/up, down.
Q8_SHAPES = [(896, 896), (128, 896), (4864, 896), (896, 4864)]
Q4_SHAPES = [(4864, 896), (896, 4864)]


def _dev(a, gpu):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(gpu)


def test_fp16_scale_conversion_exhaustive(qh, oracle, gpu):
    """Every binary16 pattern as a block scale: with s = 1 and dx = 1 the GEMV returns f16(scale) exactly."""
    import torch
    rows, cols = 65536, 32
    q = np.zeros((rows, cols), np.int8)
    q[:, 0] = 1
    scales = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    buf = np.concatenate([q.reshape(-1).view(np.uint8), scales.view(np.uint8)])
    W = qh.DeviceTensor.upload(buf, qh.Q8_0, rows, cols)
    xq = torch.zeros(cols, dtype=torch.int8, device=gpu)
    xq[0] = 1
    xd = torch.ones(1, dtype=torch.float32, device=gpu)
    got = qh.matvec_q(W, xq, xd).cpu().numpy()
    # the chain starts from acc = +0, so a -0 scale comes out as +0 (fma(-0, 1, +0) = +0) on both sides
    table = np.array([oracle.fp16_to_f32(h) for h in range(65536)], np.float32) + np.float32(0.0)
    want = oracle.matvec_q(qh.Q8_0, rows, cols, buf, np.asarray(xq.cpu()), np.asarray(xd.cpu()))
    nan = np.isnan(table)
    assert np.isnan(want[nan]).all() and np.isnan(got[nan]).all()
    assert (bits(want[~nan]) == bits(table[~nan])).all()
    bad = np.nonzero(bits(got[~nan]) != bits(want[~nan]))[0]
    assert bad.size == 0, f"{bad.size} patterns differ, first {np.arange(65536)[~nan][bad[:8]]}"


def test_quantize_q8_matches_oracle(qh, oracle, synth, gpu):
    x = synth.activations(101, 64, 896)
    # edge blocks: all zero; amax 127 (d = 1, inv = 1) with exact .5 ties of both signs, which lroundf
    # rounds away from zero; values near the top and near the bottom of the normal f32 range
    x[0, :32] = 0.0
    ties = np.arange(-15, 15, dtype=np.float32) + 0.5
    x[1, :32] = np.concatenate([[127.0, -127.0], ties]).astype(np.float32)
    x[2, :32] = -x[1, :32]
    x[3, :32] = np.linspace(-1e-30, 2e-30, 32, dtype=np.float32)
    x[4, 32:64] = 3e38
    x[4, 40] = -3e38
    q, d = qh.quantize_q8(_dev(x, gpu))
    wq, wd = oracle.quantize_q8(x)
    assert (q.cpu().numpy() == wq).all()
    assert (bits(d.cpu().numpy()) == bits(wd)).all()


@pytest.mark.parametrize("shape", Q8_SHAPES)
def test_matvec_q8_matches_oracle(qh, oracle, synth, gpu, shape):
    N, K = shape
    buf = synth.q8_tensor(1000 + N + K, N, K)
    x = synth.activations(2000 + K, 3, K)
    W = qh.DeviceTensor.upload(buf, qh.Q8_0, N, K)
    xq, xd = qh.quantize_q8(_dev(x, gpu))
    for t in range(3):
        got = qh.matvec_q(W, xq[t], xd[t]).cpu().numpy()
        want = oracle.matvec_q(qh.Q8_0, N, K, buf, xq[t].cpu().numpy(), xd[t].cpu().numpy())
        assert (bits(got) == bits(want)).all(), f"{shape} token {t}: {np.abs(got - want).max()}"


@pytest.mark.parametrize("shape", Q4_SHAPES)
def test_matvec_q4_matches_oracle(qh, oracle, synth, gpu, shape):
    N, K = shape
    buf = synth.q4_tensor(3000 + N + K, N, K)
    x = synth.activations(4000 + K, 3, K)
    W = qh.DeviceTensor.upload(buf, qh.Q4_0, N, K)
    xq, xd = qh.quantize_q8(_dev(x, gpu))
    for t in range(3):
        got = qh.matvec_q(W, xq[t], xd[t]).cpu().numpy()
        want = oracle.matvec_q(qh.Q4_0, N, K, buf, xq[t].cpu().numpy(), xd[t].cpu().numpy())
        assert (bits(got) == bits(want)).all(), f"{shape} token {t}: {np.abs(got - want).max()}"


@pytest.mark.parametrize("dtype", [2, 3])
def test_matvec_row_range_and_full_int8_range(qh, oracle, gpu, dtype):
    """Quant bytes over the whole int8 range (incl. -128, as in the reference selftest), odd row ranges."""
    import torch
    rng = np.random.default_rng(7)
    N, K = 300, 640
    qb = N * K if dtype == 2 else N * K // 2
    buf = np.concatenate([rng.integers(0, 256, qb, dtype=np.uint8),
                          (0x2000 + rng.integers(0, 0x800, N * K // 32)).astype(np.uint16).view(np.uint8)])
    x = rng.standard_normal(K).astype(np.float32)
    xq, xd = oracle.quantize_q8(x)
    W = qh.DeviceTensor.upload(buf, dtype, N, K)
    dq, dd = _dev(xq, gpu), _dev(xd, gpu)
    want = oracle.matvec_q(dtype, N, K, buf, xq, xd)
    for r0, r1 in [(0, N), (17, 18), (5, 299), (16, 48), (0, 1), (299, 300)]:
        out = torch.full((N,), 7.0, dtype=torch.float32, device=gpu)
        qh.matvec_q(W, dq, dd, out=out, r0=r0, r1=r1)
        got = out.cpu().numpy()
        assert (bits(got[r0:r1]) == bits(want[r0:r1])).all(), (r0, r1)
        assert (got[:r0] == 7.0).all() and (got[r1:] == 7.0).all(), "wrote outside [r0, r1)"


@pytest.mark.parametrize("dtype", [2, 3])
def test_matvec_vocab_sized_stream(qh, oracle, synth, gpu, dtype):
    """Vocabulary-sized matrices take the streaming kernel: whole range and ragged sub-ranges."""
    import torch
    N, K = 151936, 896
    buf = synth.q8_tensor(5000, N, K) if dtype == 2 else synth.q4_tensor(5001, N, K)
    xq, xd = oracle.quantize_q8(synth.activations(5002, 1, K)[0])
    W = qh.DeviceTensor.upload(buf, dtype, N, K)
    dq, dd = _dev(xq, gpu), _dev(xd, gpu)
    want = oracle.matvec_q(dtype, N, K, buf, xq, xd, threads=8)
    got = qh.matvec_q(W, dq, dd).cpu().numpy()
    assert (bits(got) == bits(want)).all()
    for r0, r1 in [(1, N - 3), (70001, 140003)]:
        out = torch.full((N,), 7.0, dtype=torch.float32, device=gpu)
        qh.matvec_q(W, dq, dd, out=out, r0=r0, r1=r1)
        o = out.cpu().numpy()
        assert (bits(o[r0:r1]) == bits(want[r0:r1])).all(), (r0, r1)
        assert (o[:r0] == 7.0).all() and (o[r1:] == 7.0).all()


@pytest.mark.parametrize("cols", [32, 64, 96, 4096])
def test_matvec_other_widths(qh, oracle, gpu, cols):
    rng = np.random.default_rng(cols)
    for dtype in (2, 3):
        N = 77
        qb = N * cols if dtype == 2 else N * cols // 2
        buf = np.concatenate([rng.integers(0, 256, qb, dtype=np.uint8),
                              (0x1c00 + rng.integers(0, 0x1000, N * cols // 32)).astype(np.uint16).view(np.uint8)])
        xq, xd = oracle.quantize_q8(rng.standard_normal(cols).astype(np.float32))
        W = qh.DeviceTensor.upload(buf, dtype, N, cols)
        got = qh.matvec_q(W, _dev(xq, gpu), _dev(xd, gpu)).cpu().numpy()
        want = oracle.matvec_q(dtype, N, cols, buf, xq, xd)
        assert (bits(got) == bits(want)).all(), (dtype, cols)


def test_argmax_first_max(qh, gpu):
    import torch
    x = torch.full((151936,), -float("inf"), device=gpu)
    assert int(qh.argmax(x).item()) == 0
    x[1000] = 3.0
    x[5000] = 3.0
    x[70000] = 2.0
    assert int(qh.argmax(x).item()) == 1000
    assert int(qh.argmax(x, n=1000).item()) == 0
    y = torch.randn(151936, device=gpu)
    assert int(qh.argmax(y).item()) == int(torch.argmax(y).item())
    # ragged sizes and equal maxima on both sides of a workgroup slice boundary: the lower index wins
    for n in (1, 2, 255, 2049, 4097, 1 << 22):
        z = torch.zeros(n, device=gpu)
        z[n // 2:] = 1.0
        assert int(qh.argmax(z).item()) == n // 2
    z = torch.full((1 << 22,), -1.0, device=gpu)
    z[3_000_001] = 5.0
    z[3_999_999] = 5.0
    assert int(qh.argmax(z).item()) == 3_000_001


def test_abi_rejects_bad_arguments(qh, gpu):
    import ctypes as C
    import torch
    L = qh.lib()
    out = torch.zeros(64, device=gpu)
    xq = torch.zeros(64, dtype=torch.int8, device=gpu)
    xd = torch.zeros(2, device=gpu)
    buf = torch.zeros(64 * 64 + 64 * 2 * 2, dtype=torch.uint8, device=gpu)
    bad = qh.qh_tensor(qh.F32, 64, 64, buf.data_ptr())
    assert L.qh_matvec_q(C.c_void_p(out.data_ptr()), C.byref(bad), C.c_void_p(xq.data_ptr()),
                         C.c_void_p(xd.data_ptr()), 0, 64, None) == 2
    assert b"dtype" in L.qh_last_error()
    odd = qh.qh_tensor(qh.Q8_0, 64, 48, buf.data_ptr())
    assert L.qh_matvec_q(C.c_void_p(out.data_ptr()), C.byref(odd), C.c_void_p(xq.data_ptr()),
                         C.c_void_p(xd.data_ptr()), 0, 64, None) == 3
    mis = qh.qh_tensor(qh.Q8_0, 64, 64, buf.data_ptr() + 4)
    assert L.qh_matvec_q(C.c_void_p(out.data_ptr()), C.byref(mis), C.c_void_p(xq.data_ptr()),
                         C.c_void_p(xd.data_ptr()), 0, 64, None) == 4
    ok = qh.qh_tensor(qh.Q8_0, 64, 64, buf.data_ptr())
    assert L.qh_matvec_q(C.c_void_p(out.data_ptr()), C.byref(ok), C.c_void_p(xq.data_ptr()),
                         C.c_void_p(xd.data_ptr()), 10, 65, None) == 1
    torch.cuda.synchronize()
