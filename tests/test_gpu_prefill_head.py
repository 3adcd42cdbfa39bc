"""GPU parity of the prefill matmul and the Exact Shortlist Head against the oracle.

Prefill: every (row, token) output must be bit-identical to the oracle, and to the GPU decode GEMV of
that token (the reference's own invariant, engine/src/checks.cpp:114-143).
Shortlist head: candidate set, rescored logits, coarse scores, upper bounds, tau and the greedy token
must be identical to the oracle (engine/src/model.cpp:240-334, sampler.cpp:35-37).
"""
import numpy as np
import pytest

from conftest import bits

pytestmark = pytest.mark.gpu


def _dev(a, gpu):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(gpu)


PREFILL = [(2, 896, 896), (2, 128, 896), (3, 4864, 896), (3, 896, 4864)]


@pytest.mark.parametrize("dtype,N,K", PREFILL)
@pytest.mark.parametrize("M", [1, 7, 32, 33])
def test_matmul_matches_oracle(qh, oracle, synth, gpu, dtype, N, K, M):
    buf = synth.q8_tensor(11 + N, N, K) if dtype == 2 else synth.q4_tensor(13 + N, N, K)
    x = synth.activations(17 + M, M, K)
    W = qh.DeviceTensor.upload(buf, dtype, N, K)
    xq, xd = qh.quantize_q8(_dev(x, gpu))
    got = qh.matmul_q(W, xq, xd).cpu().numpy()
    want = oracle.matmul_q(dtype, N, K, buf, xq.cpu().numpy(), xd.cpu().numpy(), threads=8)
    assert (bits(got) == bits(want)).all(), f"max diff {np.abs(got - want).max()}"


@pytest.mark.parametrize("dtype,N,K", PREFILL)
@pytest.mark.parametrize("M", [128, 512])
def test_matmul_rows_equal_gemv(qh, oracle, synth, gpu, dtype, N, K, M):
    """Large M (the 64 x 64 tile kernel): every output equals the oracle's, and every token row the decode GEMV of
    that token, bit for bit."""
    import torch
    buf = synth.q8_tensor(21 + N, N, K) if dtype == 2 else synth.q4_tensor(23 + N, N, K)
    x = synth.activations(29 + M, M, K)
    W = qh.DeviceTensor.upload(buf, dtype, N, K)
    xq, xd = qh.quantize_q8(_dev(x, gpu))
    got = qh.matmul_q(W, xq, xd)
    want = oracle.matmul_q(dtype, N, K, buf, xq.cpu().numpy(), xd.cpu().numpy(), threads=8)
    assert (bits(got.cpu().numpy()) == bits(want)).all()
    per_tok = torch.stack([qh.matvec_q(W, xq[t], xd[t]) for t in range(M)])
    assert torch.equal(got.view(torch.int32), per_tok.view(torch.int32))


def _bits_or_nan_equal(got, want):
    nan = np.isnan(want)
    assert (np.isnan(got) == nan).all(), f"{int((np.isnan(got) != nan).sum())} NaN positions differ"
    bad = np.nonzero(bits(got[~nan]) != bits(want[~nan]))[0]
    assert bad.size == 0, f"{bad.size} outputs differ, first flat indices {bad[:8]}"


@pytest.mark.parametrize("tt", ["tile", "tile32", "tile16", "tile32w8", "tile32w8:16"])
@pytest.mark.parametrize("dtype", [2, 3])
def test_matmul_tile_every_f16_scale(qh, oracle, synth, gpu, monkeypatch, tt, dtype):
    """The tile kernel's block products float(s) * d over every binary16 pattern as a row's scale (subnormals, -0,
    the largest finite values, inf and NaN), 128 tokens: NaN where the oracle has NaN, every other output bit-equal."""
    monkeypatch.setenv("QH_MM", tt)
    N, K, M = 65536, 64, 128
    buf = synth.q8_tensor(5, N, K) if dtype == 2 else synth.q4_tensor(7, N, K, group=32)
    synth.scales_of(buf, dtype, N, K).view(np.uint16)[:] = np.repeat(np.arange(65536, dtype=np.uint32)
                                                                     .astype(np.uint16), K // 32)
    W = qh.DeviceTensor.upload(buf, dtype, N, K)
    xq, xd = qh.quantize_q8(_dev(synth.activations(3, M, K), gpu))
    got = qh.matmul_q(W, xq, xd).cpu().numpy()
    want = oracle.matmul_q(dtype, N, K, buf, xq.cpu().numpy(), xd.cpu().numpy(), threads=8)
    _bits_or_nan_equal(got, want)


@pytest.mark.parametrize("tt", ["tile", "tile:8", "tile32", "tile32:8", "tile16", "tile32w8", "tile32w8:16"])
@pytest.mark.parametrize("dtype", [2, 3])
def test_matmul_tile_nonfinite_scales_by_chunk(qh, oracle, synth, gpu, monkeypatch, tt, dtype):
    """Inf and NaN row scales planted in some K chunks of some row tiles, with extreme finite scales (the largest f16,
    subnormals, negative, -0) elsewhere, at every tile variant and chunk size: every output equals the oracle's."""
    monkeypatch.setenv("QH_MM", tt)
    N, K = 200, 4864
    buf = synth.q8_tensor(41, N, K) if dtype == 2 else synth.q4_tensor(43, N, K, group=32)
    sc = synth.scales_of(buf, dtype, N, K).view(np.uint16).reshape(N, K // 32)
    for r, b, h in [(5, 9, 0x7C00), (70, 20, 0xFC00), (130, 3, 0x7E00), (131, 150, 0x7C00), (199, 151, 0xFE01),
                    (6, 10, 0x7BFF), (7, 0, 0x0001), (8, 33, 0x8000), (9, 34, 0xFBFF), (64, 70, 0x83FF),
                    (65, 71, 0x0400)]:
        sc[r, b] = h
    W = qh.DeviceTensor.upload(buf, dtype, N, K)
    for M in (130, 512):
        xq, xd = qh.quantize_q8(_dev(synth.activations(47 + M, M, K), gpu))
        got = qh.matmul_q(W, xq, xd).cpu().numpy()
        want = oracle.matmul_q(dtype, N, K, buf, xq.cpu().numpy(), xd.cpu().numpy(), threads=8)
        _bits_or_nan_equal(got, want)


def test_matmul_row_range_and_ldo(qh, oracle, synth, gpu):
    import torch
    N, K, M = 200, 896, 19
    buf = synth.q4_tensor(31, N, K)
    W = qh.DeviceTensor.upload(buf, 3, N, K)
    xq, xd = qh.quantize_q8(_dev(synth.activations(37, M, K), gpu))
    want = oracle.matmul_q(3, N, K, buf, xq.cpu().numpy(), xd.cpu().numpy())
    ldo = 300
    out = torch.full((M, ldo), 5.0, device=gpu)
    qh.matmul_q(W, xq, xd, out=out, r0=7, r1=150, ldo=ldo)
    o = out.cpu().numpy()
    assert (bits(o[:, 7:150]) == bits(want[:, 7:150])).all()
    assert (o[:, :7] == 5.0).all() and (o[:, 150:] == 5.0).all()


# ----------------------------------------------------------------------------------------- shortlist head

def _head(qh, synth, gpu, V, D, seed):
    head8, head4, err = synth.shortlist_head(seed, V, D)
    dev = (qh.DeviceTensor.upload(head8, 2, V, D), qh.DeviceTensor.upload(head4, 3, V, D),
           qh.DeviceTensor.upload(err.view(np.uint8), 1, V, D // 32))
    return (head8, head4, err), dev


def _check_head(qh, oracle, head_np, sl, xq, xd, V, D, top_k, n_valid=0, must=None):
    import torch
    head8, head4, err = head_np
    must_t = None if must is None else torch.tensor(must, dtype=torch.int32, device=xq.device)
    sl(xq, xd, n_valid=n_valid, must=must_t)
    st = sl.stats()
    o = oracle.shortlist_head(head8, head4, err, V, D, xq.cpu().numpy(), xd.cpu().numpy(), top_k=top_k,
                              n_valid=n_valid, must=must)
    assert not st["seed_tie"] and not o["seed_tie"]
    assert (bits(sl.coarse.cpu().numpy()) == bits(o["coarse"])).all(), "coarse"
    assert (bits(sl.upper.cpu().numpy()) == bits(o["upper"])).all(), "upper"
    assert st["n_rows"] == o["n_rows"] and st["n_seeds"] == o["n_seeds"]
    rows = sl.rows.cpu().numpy()[: st["n_rows"]]
    assert sorted(rows.tolist()) == sorted(o["rows"].tolist())
    assert rows[: st["n_seeds"]].tolist() == o["rows"][: o["n_seeds"]].tolist(), "seed order"
    nm = st["n_must"]
    if nm:
        assert rows[len(rows) - nm:].tolist() == o["rows"][len(o["rows"]) - nm:].tolist(), "must ids last, query order"
    assert (bits(sl.logits.cpu().numpy()) == bits(o["logits"])).all(), "logits"
    assert np.float32(st["tau"]).tobytes() == np.float32(o["tau"]).tobytes()
    nv = n_valid if 0 < n_valid < V else V
    assert st["top1"] == oracle.argmax(o["logits"], nv)
    return st, o


@pytest.mark.parametrize("top_k", [1, 20, 64, 256])
def test_shortlist_small_vocab(qh, oracle, synth, gpu, top_k):
    V, D = 6007, 896
    head_np, (h8, h4, he) = _head(qh, synth, gpu, V, D, 41)
    sl = qh.ShortlistHead(h8, h4, he, top_k=top_k)
    x = synth.activations(43, 6, D, scale=0.5)
    xq, xd = qh.quantize_q8(_dev(x, gpu))
    for t in range(4):
        _check_head(qh, oracle, head_np, sl, xq[t], xd[t], V, D, top_k)
    # n_valid below V and must ids (duplicates, out-of-range and >= n_valid ones are ignored)
    must = [5, 17, 5, 6000, -3, 4000, 123, 17]
    _check_head(qh, oracle, head_np, sl, xq[4], xd[4], V, D, top_k, n_valid=5000, must=must)
    _check_head(qh, oracle, head_np, sl, xq[5], xd[5], V, D, top_k, n_valid=5000, must=must)


@pytest.mark.parametrize("top_k", [1, 20])
def test_shortlist_long_must_list(qh, oracle, synth, gpu, top_k):
    """A history-sized must list: 3000 ids with many repeats and some out of range. Every first occurrence of a valid
    id comes back exact, listed last in query order, as the oracle lists them."""
    V, D = 6007, 896
    head_np, (h8, h4, he) = _head(qh, synth, gpu, V, D, 41)
    sl = qh.ShortlistHead(h8, h4, he, top_k=top_k)
    x = synth.activations(71, 2, D, scale=0.5)
    xq, xd = qh.quantize_q8(_dev(x, gpu))
    rng = np.random.default_rng(5)
    must = rng.integers(-20, V + 20, 3000)
    must[rng.random(3000) < 0.5] = must[0]
    for t, n_valid in ((0, 0), (1, 5500)):
        st, o = _check_head(qh, oracle, head_np, sl, xq[t], xd[t], V, D, top_k, n_valid=n_valid, must=must.tolist())
        nm = st["n_must"]
        nv = n_valid if n_valid else V
        _, first = np.unique(must, return_index=True)
        expect = [int(must[i]) for i in sorted(first) if 0 <= must[i] < nv]
        assert nm == len(expect) > 100
        rows = sl.rows.cpu().numpy()
        n = st["n_rows"]
        assert rows[n - nm:n].tolist() == expect == o["rows"][-nm:].tolist()
    # the same list again with an empty window (the kernels reset what the previous query left)
    _check_head(qh, oracle, head_np, sl, xq[0], xd[0], V, D, top_k)


def _cluster_head(synth, V, D, seed, r0, n, x):
    """A random Q8_0 head whose rows [r0, r0 + n) share one code pattern aligned with x, with consecutive f16 scales:
    their scores rise row by row far above the rest, so the best keys crowd a few screen shares. The codes are
    multiples of 8 in [-56, 56] with -64 first in every block, so the 4-bit copy is exact (scale 8 d, zero error) and
    no two coarse scores of the cluster tie."""
    head8 = synth.q8_tensor(seed, V, D)
    q = head8[: V * D].view(np.int8).reshape(V, D)
    d = head8[V * D:].view(np.float16).reshape(V, D // 32)
    c = (np.clip(np.rint(x / np.abs(x).max() * 7.0), -7, 7) * 8).astype(np.int8)
    c[::32] = -64
    q[r0:r0 + n] = c
    first = int(np.float16(1e-3).view(np.uint16))
    d[r0:r0 + n] = np.arange(first, first + n, dtype=np.uint16).view(np.float16)[:, None]
    head4, err = synth.shortlist_copy(head8, V, D)
    return head8, head4, err


def _decoy_head(synth, V, D, seed, x, n_decoy, factor):
    """A random Q8_0 head with its 4-bit copy, where n_decoy rows that score well below the best (ranks 40 on under the
    exact head for the hidden state x, dequantized) get 4-bit scales `factor` times too large, their error bounds
    recomputed from the real difference (rounded up to f16, as synth.shortlist_copy does). Their coarse scores then
    lead, so they are the seeds, and their exact logits (the k-th best of which is tau) sit far below their coarse
    scores: the rows with tau <= upper bound < the select kernel's speculative cut need the second rescoring pass."""
    head8 = synth.q8_tensor(seed, V, D)
    head4, err = synth.shortlist_copy(head8, V, D)
    w = synth.dequant_q8(head8, V, D)
    decoys = np.argsort(-(w @ x))[40:40 + n_decoy]
    nb = D // 32
    s4 = head4[V * D // 2:].view(np.float16).reshape(V, nb)
    nib = head4[:V * D // 2].reshape(V, nb, 16)
    codes = np.concatenate([nib & 15, nib >> 4], axis=2).astype(np.float64) - 8.0  # [V][block][32], element order
    for r in decoys:
        s4[r] = (s4[r].astype(np.float32) * factor).astype(np.float16)
        diff = codes[r] * s4[r].astype(np.float64)[:, None] - w[r].reshape(nb, 32).astype(np.float64)
        e = np.sqrt((diff * diff).sum(axis=1))
        e16 = e.astype(np.float16)
        low = e16.astype(np.float64) < e
        e16[low] = np.nextafter(e16[low], np.float16(np.inf))
        err[r] = e16
    return head8, head4, err, decoys


@pytest.mark.parametrize("top_k", [1, 20])
def test_shortlist_second_rescoring_pass(qh, oracle, synth, gpu, top_k):
    """tau below the speculative cut (the seeds' 4-bit copies overstate them): the rows with tau <= upper < cut, which
    the first pass leaves out, are rescored in the second, and every output equals the oracle's bit for bit."""
    V, D = 6007, 896
    x = synth.activations(43, 1, D, scale=0.5)
    xq, xd = oracle.quantize_q8(x)
    xf = (xq[0].reshape(-1, 32).astype(np.float32) * xd[0][:, None]).reshape(-1)
    head8, head4, err, decoys = _decoy_head(synth, V, D, 41, xf, top_k + 12, 2.0)
    o = oracle.shortlist_head(head8, head4, err, V, D, xq[0], xd[0], top_k=top_k)
    # the case on the CPU: every seed a decoy, tau below the cut, rows between them
    ck = np.sort(o["coarse"])[::-1][top_k - 1]
    cut = np.float32(ck - (np.float32(abs(ck)) * np.float32(0.0625) + np.float32(1e-3)))
    tau = np.float32(o["tau"])
    assert np.isin(o["rows"][:o["n_seeds"]], decoys).all()
    assert tau < cut and ((o["upper"] >= tau) & (o["upper"] < cut)).sum() > 100
    dev = (qh.DeviceTensor.upload(head8, 2, V, D), qh.DeviceTensor.upload(head4, 3, V, D),
           qh.DeviceTensor.upload(err.view(np.uint8), 1, V, D // 32))
    sl = qh.ShortlistHead(*dev, top_k=top_k)
    xq_d, xd_d = qh.quantize_q8(_dev(x, gpu))
    st, _ = _check_head(qh, oracle, (head8, head4, err), sl, xq_d[0], xd_d[0], V, D, top_k)
    assert st["n_rows"] == o["n_rows"] > 500


@pytest.mark.parametrize("top_k,r0,n", [(1, 70001, 300), (20, 5, 700), (55, 40000, 9600), (256, 90000, 9600)])
def test_shortlist_crowded_shares(qh, oracle, synth, gpu, top_k, r0, n):
    """The best keys crowd a few screen shares: each share publishes only its best four keys, so shares holding more
    than four of them are read again (a few hundred keys), and past 1024 keys at or above the cut the selection falls
    back to a radix select over the selected shares' rows (55: about 9,300 keys)."""
    V, D = 151936, 896
    x = synth.activations(211, 1, D, scale=0.5)
    head_np = _cluster_head(synth, V, D, 209, r0, n, x[0])
    h8, h4, he = (qh.DeviceTensor.upload(head_np[0], 2, V, D), qh.DeviceTensor.upload(head_np[1], 3, V, D),
                  qh.DeviceTensor.upload(head_np[2].view(np.uint8), 1, V, D // 32))
    sl = qh.ShortlistHead(h8, h4, he, top_k=top_k)
    xq, xd = qh.quantize_q8(_dev(x, gpu))
    st, o = _check_head(qh, oracle, head_np, sl, xq[0], xd[0], V, D, top_k)
    assert r0 + n - top_k - 8 <= min(sl.rows[: st["n_seeds"]].cpu().numpy().tolist())  # the cluster's last rows
    must = [r0 + n - 1, r0 + n - 3, 17, r0 + n - 1]  # the best rows as must ids: not seeds, listed last
    _check_head(qh, oracle, head_np, sl, xq[0], xd[0], V, D, top_k, must=must)


def test_shortlist_fewer_shares_than_seeds(qh, oracle, synth, gpu):
    """A vocabulary of a few screen shares (fewer than top_k + 9): every eligible row is a seed candidate."""
    V, D = 300, 896
    head_np, (h8, h4, he) = _head(qh, synth, gpu, V, D, 223)
    x = synth.activations(227, 2, D, scale=0.5)
    xq, xd = qh.quantize_q8(_dev(x, gpu))
    for top_k in (1, 20, 55, 64, 256):
        sl = qh.ShortlistHead(h8, h4, he, top_k=top_k)
        _check_head(qh, oracle, head_np, sl, xq[0], xd[0], V, D, top_k)
        _check_head(qh, oracle, head_np, sl, xq[1], xd[1], V, D, top_k, n_valid=250, must=[3, 299, 3, 7])


@pytest.mark.parametrize("top_k", [64, 128, 256])
def test_shortlist_large_topk_full_vocab(qh, oracle, synth, gpu, top_k):
    """The benchmark head's shape at the top-k values of sampling (more seeds than a wave's lanes: the cut from a radix
    select over the published keys, tau over the workgroup, the seeds as band bits), with and without must ids:
    everything equals the oracle bit for bit, and the reference build's own Model::shortlist_head returns the same
    rows and logits."""
    import oracle as orc
    V, D = 151936, 896
    head_np, (h8, h4, he) = _head(qh, synth, gpu, V, D, 47)
    sl = qh.ShortlistHead(h8, h4, he, top_k=top_k)
    x = synth.activations(59, 3, D, scale=0.5)
    xq, xd = qh.quantize_q8(_dev(x, gpu))
    must = np.random.default_rng(61).integers(0, V, 500).tolist()
    for t, mu in ((0, None), (1, None), (2, must)):
        print(f"large top-k {top_k}, vector {t}", flush=True)
        st, o = _check_head(qh, oracle, head_np, sl, xq[t], xd[t], V, D, top_k, must=mu)
        assert st["n_seeds"] == top_k + 8
        if orc.ref is not None:
            r = orc.ref.shortlist_head(*head_np, V, D, xq[t].cpu().numpy(), xd[t].cpu().numpy(), top_k=top_k, must=mu,
                                       threads=8)
            assert r["n_rows"] == st["n_rows"]
            assert sorted(r["rows"].tolist()) == sorted(sl.rows.cpu().numpy()[: st["n_rows"]].tolist())
            assert (bits(r["logits"]) == bits(sl.logits.cpu().numpy())).all()


def test_shortlist_full_vocab(qh, oracle, synth, gpu):
    """The benchmark head: vocab 151936 x 896, k = 1, a few hidden states N(0,1)*0.5."""
    V, D = 151936, 896
    head_np, (h8, h4, he) = _head(qh, synth, gpu, V, D, 47)
    sl = qh.ShortlistHead(h8, h4, he, top_k=1)
    x = synth.activations(53, 4, D, scale=0.5)
    xq, xd = qh.quantize_q8(_dev(x, gpu))
    full = qh.matvec_q(h8, xq[0], xd[0])
    for t in range(4):
        st, o = _check_head(qh, oracle, head_np, sl, xq[t], xd[t], V, D, 1)
        assert 0 < st["n_rows"] < V // 10
    # the top-1 of the shortlist is the top-1 of the full 8-bit head, and its logit is bit-identical
    sl(xq[0], xd[0])
    st = sl.stats()
    assert st["top1"] == int(qh.argmax(full).item())
    assert np.float32(st["top1_logit"]).tobytes() == full[st["top1"]].cpu().numpy().tobytes()


@pytest.mark.parametrize("tt", ["stage", "stage:2", "stage:3", "stage:4", "tile", "tile32", "tile32:8"])
@pytest.mark.parametrize("K", [512, 1536, 2560, 3584, 5632, 8192])
@pytest.mark.parametrize("dtype", [2, 3])
def test_matmul_staged_chunk_counts(qh, oracle, synth, gpu, monkeypatch, tt, dtype, K):
    """The LDS-staged kernel at every chunk count it plans for (16 blocks a chunk): one chunk, the straight-line short
    rows, all chunks held in registers (4 / 6 / 8 / 12 sets, odd counts with a clamped spare) and the refilled
    2 / 3 / 4 set pipeline past that."""
    monkeypatch.setenv("QH_MM", tt)
    N = 40
    buf = synth.q8_tensor(83 + K, N, K) if dtype == 2 else synth.q4_tensor(89 + K, N, K)
    W = qh.DeviceTensor.upload(buf, dtype, N, K)
    for M in (1, 17, 40):
        xq, xd = qh.quantize_q8(_dev(synth.activations(97 + M, M, K), gpu))
        got = qh.matmul_q(W, xq, xd).cpu().numpy()
        want = oracle.matmul_q(dtype, N, K, buf, xq.cpu().numpy(), xd.cpu().numpy(), threads=8)
        assert (bits(got) == bits(want)).all(), (tt, M)


@pytest.mark.parametrize("tt", ["stage", "tile", "tile:8", "tile32", "tile32:8", "tile16", "tile32w8", "tile32w8:16", "lds:1", "lds:2", "lds:4", "reg:1:1",
                                "reg:1:4", "reg:2:2", "reg:4:1", "reg:4:4"])
@pytest.mark.parametrize("dtype,N,K", [(2, 200, 896), (3, 200, 896), (2, 40, 4864), (3, 40, 4864)])
def test_matmul_every_token_tiling(qh, oracle, synth, gpu, monkeypatch, tt, dtype, N, K):
    """Both prefill kernels at every token tiling (LDS-staged block sums, register chains) on ragged shapes: rows not a
    multiple of 16, a last K chunk shorter than the others, token counts around the tile widths."""
    monkeypatch.setenv("QH_MM", tt)
    buf = synth.q8_tensor(61 + N, N, K) if dtype == 2 else synth.q4_tensor(67 + N, N, K)
    W = qh.DeviceTensor.upload(buf, dtype, N, K)
    for M in (1, 15, 17, 40, 65, 130):
        xq, xd = qh.quantize_q8(_dev(synth.activations(71 + M, M, K), gpu))
        got = qh.matmul_q(W, xq, xd).cpu().numpy()
        want = oracle.matmul_q(dtype, N, K, buf, xq.cpu().numpy(), xd.cpu().numpy(), threads=8)
        assert (bits(got) == bits(want)).all(), (tt, M)
