"""Pins the oracle (oracle/quanta_oracle.c) before any GPU result is compared with it.

Three independent sources, chosen so that a plausible slip in the oracle fails at least one:
  * golden vectors written by the reference's own kernels, compiled from its sources
    (tests/golden/*.npz, made by tests/golden/make_golden.py);
  * the reference build itself (oracle/_ref), where it is present, on fresh seeded inputs;
  * what the mathematics fixes: IEEE binary16 decoding checked against numpy's conversion for all 65,536
    patterns; quantize_q8's ties-away-from-zero and its +-127 end points; every GEMV output recomputed
    in exact rational arithmetic with one correctly rounded f32 operation per step, in the reference's
    association, which the other associations provably fail; the shortlist's bound, exactness and
    top-k invariants (reference engine/src/checks.cpp:178-239).
No GPU is used.
"""
import os
from fractions import Fraction

import numpy as np
import pytest

from conftest import GOLDEN, bits

Q8_0, Q4_0 = 2, 3


def golden(name):
    path = os.path.join(GOLDEN, name)
    if not os.path.exists(path):
        pytest.fail(f"{path} is missing (python tests/golden/make_golden.py)")
    return np.load(path, allow_pickle=False)


# ------------------------------------------------------------------ exact f32 arithmetic on rationals

def f32_round(x: Fraction) -> Fraction:
    """x rounded to the nearest binary32 value, ties to even (no overflow handling: inputs stay small)."""
    if x == 0:
        return Fraction(0)
    sign = -1 if x < 0 else 1
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    quantum = Fraction(2) ** (max(e, -126) - 23)
    q = a / quantum
    n = q.numerator // q.denominator
    rem = q - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return sign * n * quantum


def exact_rows(codes: np.ndarray, scales: np.ndarray, xq: np.ndarray, xd: np.ndarray, assoc: str) -> np.ndarray:
    """Per-row chain over 32-blocks with exact integer block sums, every f32 step correctly rounded.

    assoc "ref":   p = rnd(s * dw); acc = rnd(p * dx + acc)      (fused multiply-add, the reference build)
    assoc "split": acc = rnd(acc + rnd(p * dx))                   (no fusion)
    assoc "swap":  acc = rnd(s * rnd(dw * dx) + acc)              (scales multiplied first)
    """
    rows, cols = codes.shape
    nb = cols // 32
    s = (codes.reshape(rows, nb, 32).astype(np.int64) * xq.reshape(nb, 32).astype(np.int64)).sum(axis=2)
    dx = [Fraction(float(v)) for v in xd]
    out = np.empty(rows, np.float32)
    for r in range(rows):
        acc = Fraction(0)
        for b in range(nb):
            dw = Fraction(float(scales[r, b]))
            sb = Fraction(int(s[r, b]))
            if assoc == "ref":
                acc = f32_round(f32_round(sb * dw) * dx[b] + acc)
            elif assoc == "split":
                acc = f32_round(acc + f32_round(f32_round(sb * dw) * dx[b]))
            else:
                acc = f32_round(sb * f32_round(dw * dx[b]) + acc)
        out[r] = np.float32(float(acc))
    return out


def decode(buf: np.ndarray, dtype: int, rows: int, cols: int):
    """Codes [rows][cols] and f32 scales [rows][cols/32] from .qnt bytes (written independently of the
    oracle: element j of a Q4_0 block is the low nibble of byte j, element 16 + j its high nibble)."""
    if dtype == Q8_0:
        codes = buf[: rows * cols].view(np.int8).reshape(rows, cols)
        qb = rows * cols
    else:
        p = buf[: rows * cols // 2].reshape(rows * cols // 32, 16)
        codes = np.concatenate([(p & 15).astype(np.int16) - 8, (p >> 4).astype(np.int16) - 8], axis=1)
        codes = codes.reshape(rows, cols)
        qb = rows * cols // 2
    sc = buf[qb: qb + rows * cols // 32 * 2].view(np.float16).astype(np.float32).reshape(rows, cols // 32)
    return codes, sc


# ------------------------------------------------------------------ binary16 and activation quantization

def test_fp16_to_f32_all_patterns(oracle):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([oracle.fp16_to_f32(int(v)) for v in h], np.float32)
    nan = np.isnan(want)
    assert nan.sum() == 2 * 1023 and np.isnan(got[nan]).all()
    assert (bits(got[~nan]) == bits(want[~nan])).all()


def test_quantize_q8_golden(oracle):
    g = golden("kernels.npz")
    q, d = oracle.quantize_q8(g["qx_in"])
    assert (q == g["qx_q"]).all()
    assert (bits(d) == bits(g["qx_d"])).all()


def test_quantize_q8_rounding_and_range(oracle):
    # amax = 127 gives d = 1 and inv = 1, so q is the value itself rounded half away from zero
    ties = np.arange(-15, 15, dtype=np.float32) + 0.5
    x = np.concatenate([[127.0, -127.0], ties]).astype(np.float32)
    q, d = oracle.quantize_q8(x)
    assert d[0] == 1.0
    assert (q[2:] == np.where(ties > 0, np.floor(ties) + 1, np.ceil(ties) - 1)).all()
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((64, 256)) * np.exp(rng.uniform(-20, 20, (64, 1)))).astype(np.float32)
    q, d = oracle.quantize_q8(x)
    xb, qb = x.reshape(64, 8, 32), q.reshape(64, 8, 32).astype(np.int32)
    amax = np.abs(xb).max(axis=2)
    assert (bits(d) == bits((amax / np.float32(127)).astype(np.float32))).all()
    assert (np.abs(qb) <= 127).all()
    # the element of largest magnitude maps to +-127 and every code is within half a step of x / d
    top = np.take_along_axis(qb, np.abs(xb).argmax(axis=2)[..., None], 2)[..., 0]
    assert (np.abs(top) == 127).all()
    err = np.abs(qb * d[..., None].astype(np.float64) - xb)
    assert (err <= 0.5 * d[..., None] * (1 + 1e-6) + 1e-45).all()
    z, dz = oracle.quantize_q8(np.zeros(64, np.float32))
    assert (z == 0).all() and (dz == 0).all()


# ------------------------------------------------------------------ GEMV and prefill matmul

KERNEL_CASES = [(dt, name, r, c) for dt, name in ((Q8_0, "q8"), (Q4_0, "q4")) for r, c in ((48, 896), (16, 4864))]


@pytest.mark.parametrize("dtype,name,rows,cols", KERNEL_CASES)
def test_matvec_golden(oracle, dtype, name, rows, cols):
    g = golden("kernels.npz")
    key = f"{name}_{rows}x{cols}"
    for t in range(2):
        got = oracle.matvec_q(dtype, rows, cols, g[f"{key}_w"], g[f"{key}_xq"][t], g[f"{key}_xd"][t])
        assert (bits(got) == bits(g[f"{key}_out"][t])).all()


@pytest.mark.parametrize("dtype,name", [(Q8_0, "q8"), (Q4_0, "q4")])
def test_matvec_exact_arithmetic(oracle, dtype, name):
    """Each output equals the reference association evaluated exactly, and the alternatives do not."""
    g = golden("kernels.npz")
    key = f"{name}_48x896"
    w, xq, xd = g[f"{key}_w"], g[f"{key}_xq"][0], g[f"{key}_xd"][0]
    codes, sc = decode(w, dtype, 48, 896)
    got = oracle.matvec_q(dtype, 48, 896, w, xq, xd)
    assert (bits(got) == bits(exact_rows(codes, sc, xq, xd, "ref"))).all()
    for other in ("split", "swap"):
        assert (bits(got) != bits(exact_rows(codes, sc, xq, xd, other))).any(), other


@pytest.mark.parametrize("dtype,name", [(Q8_0, "q8"), (Q4_0, "q4")])
def test_matmul_golden_and_rows_equal_matvec(oracle, dtype, name):
    g = golden("kernels.npz")
    w, xq, xd, want = g[f"{name}_mm_w"], g[f"{name}_mm_xq"], g[f"{name}_mm_xd"], g[f"{name}_mm_out"]
    got = oracle.matmul_q(dtype, 40, 256, w, xq, xd)
    assert (bits(got) == bits(want)).all()
    for t in range(xq.shape[0]):
        assert (bits(got[t]) == bits(oracle.matvec_q(dtype, 40, 256, w, xq[t], xd[t]))).all()
    band = oracle.matmul_q(dtype, 40, 256, w, xq, xd, r0=9, r1=33)
    assert (bits(band[:, 9:33]) == bits(want[:, 9:33])).all() and (band[:, :9] == 0).all()


def test_reference_selftest_fixture(oracle):
    """The reference's own kernel_selftest data (checks.cpp:64-146), regenerated from its xorshift recipe."""
    import hashlib
    from golden.selftest_fixture import selftest_inputs
    g = golden("selftest.npz")

    def sha(*arrays):
        h = hashlib.sha256()
        for a in arrays:
            h.update(np.ascontiguousarray(a).view(np.uint8).tobytes())
        return h.hexdigest()

    for dtype, name, fx in selftest_inputs():
        assert sha(fx["w"]) == str(g[f"{name}_w_sha"]) and sha(fx["x"], fx["xs"]) == str(g[f"{name}_x_sha"])
        q, d = oracle.quantize_q8(fx["x"])
        assert (q == g[f"{name}_xq"]).all() and (bits(d) == bits(g[f"{name}_xd"])).all()
        mv = oracle.matvec_q(dtype, 4864, 896, fx["w"], q, d, threads=8)
        want = g[f"{name}_matvec"]
        assert (bits(mv) == bits(want)).all()
        # the reference's own acceptance criterion, trivially met by an exact result
        assert np.abs(mv.astype(np.float64) - want).max() / np.abs(want).max() < 1e-4
        qs, ds = oracle.quantize_q8(fx["xs"])
        assert sha(qs, ds) == str(g[f"{name}_xs_q_sha"])
        assert sha(oracle.matmul_q(dtype, 4864, 896, fx["w"], qs, ds, threads=8)) == str(g[f"{name}_matmul32_sha"])
        assert sha(oracle.matmul_q(dtype, 4864, 896, fx["w"], qs[:7], ds[:7], threads=8)) == \
            str(g[f"{name}_matmul7_sha"])


# ------------------------------------------------------------------ shortlist head

def shortlist_queries():
    g = golden("shortlist.npz")
    V, D = int(g["V"]), int(g["D"])
    for i in range(5):
        must = g[f"q{i}_must"]
        yield g, V, D, i, int(g[f"q{i}_topk"]), int(g[f"q{i}_nvalid"]), (must.tolist() if must.size else None)


def test_shortlist_golden(oracle):
    for g, V, D, i, k, nv, must in shortlist_queries():
        o = oracle.shortlist_head(g["head8"], g["head4"], g["err"], V, D, g[f"q{i}_xq"], g[f"q{i}_xd"], top_k=k,
                                  n_valid=nv, must=must)
        assert not o["seed_tie"]
        for f in ("logits", "coarse", "upper"):
            assert (bits(o[f]) == bits(g[f"q{i}_{f}"])).all(), (i, f)
        want = g[f"q{i}_rows"]
        assert o["n_rows"] == int(g[f"q{i}_nrows"]) == want.size
        ns = o["n_seeds"]
        assert ns == k + 8
        # the reference's seed order comes from nth_element; candidates and must ids follow in a fixed order
        assert sorted(o["rows"][:ns].tolist()) == sorted(want[:ns].tolist())
        assert o["rows"][ns:].tolist() == want[ns:].tolist()
        assert 0 < o["n_rows"] < V


def test_shortlist_invariants(oracle):
    """The reference's check_head invariants (checks.cpp:178-239) against the full 8-bit head."""
    for g, V, D, i, k, nv, must in shortlist_queries():
        xq, xd = g[f"q{i}_xq"], g[f"q{i}_xd"]
        o = oracle.shortlist_head(g["head8"], g["head4"], g["err"], V, D, xq, xd, top_k=k, n_valid=nv, must=must)
        full = oracle.matvec_q(Q8_0, V, D, g["head8"], xq, xd)
        coarse4 = oracle.matvec_q(Q4_0, V, D, g["head4"], xq, xd)
        assert (bits(o["coarse"]) == bits(coarse4)).all()
        bound = o["upper"] - o["coarse"]
        assert (np.abs(full - o["coarse"]) <= bound).all(), "error bound violated"
        ex = o["logits"] != -np.inf
        assert (bits(o["logits"][ex]) == bits(full[ex])).all()
        n = nv if nv else V
        order = np.argsort(-full[:n], kind="stable")
        assert ex[order[:k]].all(), "true top-k not rescored"
        for m in must or []:
            if 0 <= m < n:
                assert ex[m]
        assert oracle.argmax(o["logits"], n) == oracle.argmax(full, n)


def test_shortlist_tie_rule(oracle, synth):
    """Equal coarse scores: the lower row wins the seed slot, and a tie at the cut is flagged."""
    V, D = 40, 64
    head8 = synth.q8_tensor(3, V, D)
    head8[: V * D] = np.tile(head8[:D], V)   # every row has the same codes ...
    head8[V * D:] = np.tile(head8[V * D: V * D + 4], V)  # ... and the same scales
    head4, err = synth.shortlist_copy(head8, V, D)
    xq, xd = oracle.quantize_q8(synth.activations(4, 1, D)[0])
    o = oracle.shortlist_head(head8, head4, err, V, D, xq, xd, top_k=1)
    assert o["n_seeds"] == 9 and o["rows"][:9].tolist() == list(range(9))
    assert o["seed_tie"]


# ------------------------------------------------------------------ against the reference build itself

@pytest.fixture(scope="module")
def ref():
    import oracle as o
    if o.ref is None:
        pytest.skip("oracle/_ref is not built (the reference sources are not mounted here)")
    return o.ref


def test_oracle_equals_reference_build(oracle, ref, synth):
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((16, 4864)) * np.exp(rng.uniform(-8, 8, (16, 1)))).astype(np.float32)
    for t in range(16):
        q, d = oracle.quantize_q8(x[t])
        rq, rd = ref.quantize_q8(x[t])
        assert (q == rq).all() and (bits(d) == bits(rd)).all()
    for dtype, (n, k) in [(Q8_0, (896, 896)), (Q8_0, (128, 896)), (Q8_0, (4864, 896)), (Q8_0, (896, 4864)),
                          (Q4_0, (4864, 896)), (Q4_0, (896, 4864))]:
        w = synth.q8_tensor(n + k, n, k) if dtype == Q8_0 else synth.q4_tensor(n + k, n, k)
        q, d = oracle.quantize_q8(synth.activations(k, 33, k))
        assert (bits(oracle.matvec_q(dtype, n, k, w, q[0], d[0])) ==
                bits(ref.matvec_q(dtype, n, k, w, q[0], d[0], threads=4))).all()
        assert (bits(oracle.matmul_q(dtype, n, k, w, q, d, threads=4)) ==
                bits(ref.matmul_q(dtype, n, k, w, q, d, threads=4))).all()


def test_oracle_shortlist_equals_reference_build(oracle, ref, synth):
    V, D = 20011, 896
    head8, head4, err = synth.shortlist_head(19, V, D)
    x = synth.activations(23, 4, D, scale=0.5)
    for t, (k, nv, must) in enumerate([(1, 0, None), (20, 0, None), (1, 19000, [3, 3, 19500, 7000]),
                                       (5, 0, [1, 2, 3])]):
        q, d = oracle.quantize_q8(x[t])
        o = oracle.shortlist_head(head8, head4, err, V, D, q, d, top_k=k, n_valid=nv, must=must)
        r = ref.shortlist_head(head8, head4, err, V, D, q, d, top_k=k, n_valid=nv, must=must, threads=8)
        assert not o["seed_tie"]
        for f in ("logits", "coarse", "upper"):
            assert (bits(o[f]) == bits(r[f])).all(), f
        assert o["n_rows"] == r["n_rows"]
        ns = o["n_seeds"]
        assert sorted(o["rows"][:ns].tolist()) == sorted(r["rows"][:ns].tolist())
        assert o["rows"][ns:].tolist() == r["rows"][ns:].tolist()


# ------------------------------------------------------------------ unquantized weights (matvec_ref, get_row)

F32, F16 = 0, 1


def _dense(seed, rows, cols, dtype):
    w = (np.random.default_rng(seed).standard_normal((rows, cols)) * 0.05).astype(np.float32)
    return w.astype(np.float16).view(np.uint8).reshape(-1) if dtype == F16 else w.view(np.uint8).reshape(-1)


def _dense_values(buf, rows, cols, dtype):
    return (buf.view(np.float16) if dtype == F16 else buf.view(np.float32)).astype(np.float32).reshape(rows, cols)


@pytest.mark.parametrize("dtype", [F32, F16])
def test_matvec_f_exact_arithmetic(oracle, dtype):
    """matvec_ref (ops_ref.cpp:8-27): each output is the chain acc = rnd(w_i x_i + acc) from +0 in column order (the
    build's multiply-add contraction), evaluated exactly; the unfused chain rnd(acc + rnd(w_i x_i)) differs."""
    rows, cols = 12, 160
    buf = _dense(5 + dtype, rows, cols, dtype)
    x = (np.random.default_rng(7).standard_normal(cols) * np.exp(np.random.default_rng(8).uniform(-3, 3, cols)))
    x = x.astype(np.float32)
    got = oracle.matvec_f(dtype, rows, cols, buf, x)
    w = _dense_values(buf, rows, cols, dtype)
    fused, split = np.empty(rows, np.float32), np.empty(rows, np.float32)
    for r in range(rows):
        a = b = Fraction(0)
        for i in range(cols):
            p = Fraction(float(w[r, i])) * Fraction(float(x[i]))
            a = f32_round(p + a)
            b = f32_round(b + f32_round(p))
        fused[r], split[r] = np.float32(float(a)), np.float32(float(b))
    assert (bits(got) == bits(fused)).all()
    assert (bits(got) != bits(split)).any()
    band = oracle.matvec_f(dtype, rows, cols, buf, x, r0=3, r1=9)
    assert (bits(band[3:9]) == bits(fused[3:9])).all() and (band[:3] == 0).all() and (band[9:] == 0).all()


def test_get_row_every_dtype(oracle, synth):
    """get_row (ops_ref.cpp:162-192) against an independent dequantization of the .qnt bytes."""
    rows, cols = 9, 256
    for dtype in (F32, F16):
        buf = _dense(3, rows, cols, dtype)
        want = _dense_values(buf, rows, cols, dtype)
        for r in (0, 4, 8):
            assert (bits(oracle.get_row(dtype, rows, cols, buf, r)) == bits(want[r])).all()
    for dtype in (Q8_0, Q4_0):
        buf = synth.q8_tensor(3, rows, cols) if dtype == Q8_0 else synth.q4_tensor(3, rows, cols)
        codes, sc = decode(buf, dtype, rows, cols)
        want = codes.astype(np.float32) * np.repeat(sc, 32, axis=1)
        for r in (0, 4, 8):
            assert (bits(oracle.get_row(dtype, rows, cols, buf, r)) == bits(want[r])).all()


def test_oracle_dense_equals_reference_build(oracle, ref, synth):
    """qo_matvec_f and qo_get_row against the reference's own matvec_ref (through Model::linear's row split) and
    get_row, at the decoder's shapes."""
    for dtype in (F32, F16):
        for n, k in [(896, 896), (128, 896), (4864, 896), (896, 4864)]:
            buf = _dense(n + k + dtype, n, k, dtype)
            x = synth.activations(k + dtype, 1, k)[0]
            assert (bits(oracle.matvec_f(dtype, n, k, buf, x)) == bits(ref.matvec_f(dtype, n, k, buf, x, threads=4))).all()
    for dtype in (F32, F16, Q8_0, Q4_0):
        rows, cols = 300, 896
        buf = (_dense(17, rows, cols, dtype) if dtype in (F32, F16) else
               synth.q8_tensor(17, rows, cols) if dtype == Q8_0 else synth.q4_tensor(17, rows, cols))
        for r in (0, 151, 299):
            assert (bits(oracle.get_row(dtype, rows, cols, buf, r)) == bits(ref.get_row(dtype, rows, cols, buf, r))).all()
