"""GPU parity of sampling mode, through the C-ABI.

* qh_sample (Sampler::sample, sampler.cpp:22-85) against the oracle's restatement (itself pinned against the
  reference's Sampler in test_sampler.py): the chosen id and the generator state, over the parameter space, chained
  draws, full-vocabulary candidates (the pool-overflow path included) and the shortlist head's row list;
* qh_sample_ws with more survivors than one workgroup holds (top_k 0, or above 256: the radix-sorted path), over
  vocabularies up to 151936 ids and over the head's row list;
* the decoder with head queries from the session's sampler parameters (must ids = the history window) and Sampler
  draws, on a small model against the oracle session (itself pinned against the reference's Session in
  test_sampling_session.py), for the chat flow, `gen` with sampling options and greedy-with-penalty, eager and with
  one step captured in a HIP graph and replayed; top_k 0 (the full head, every id a survivor) and, on a model without
  the shortlist tensors, top_k 300;
* the benchmark model (24 layers, vocab 151936, 512-id prompt): 256 tokens of the chat flow (temperature 0.7, top-k
  20, top-p 0.8, penalty 1.1, seed 0x51A7C0DE) and of `gen --top-k 20 --repeat-penalty 1.1` equal the reference
  Session's streams (tests/golden/e2e_sampled.npz), with every step's 8-bit head rows.
"""
import os

import numpy as np
import pytest

import oracle as oracle_mod
from conftest import GOLDEN
from decoder_util import oracle_decoder, oracle_session, qnt_module

pytestmark = pytest.mark.gpu


def _params(qh, t):
    return qh.qh_sampler_params(*t), oracle_mod.SamplerParams(*t)


def _state_dev(state, device):
    import torch
    return torch.tensor(np.array([state], np.uint64).view(np.int64), device=device)


def _state_host(t):
    return int(t.cpu().numpy().view(np.uint64)[0])


def _draws(qh, oracle, logits, n_valid, hist, t, seed, n_draws, head=None, ws=None):
    import torch
    dev = logits.device
    pq, po = _params(qh, t)
    st = oracle.sampler_seed(seed)
    sd = _state_dev(st, dev)
    hd = torch.tensor(np.asarray(hist, np.int32), device=dev) if len(hist) else None
    host = logits.cpu().numpy()
    for d in range(n_draws):
        got = int(qh.sample(logits, pq, sd, hd, n_valid=n_valid, head=head, ws=ws).cpu().item())
        want, _, st = oracle.sample(host, n_valid, hist, po, st)
        assert got == want, (t, d)
        assert _state_host(sd) == st, (t, d)


def test_sample_equals_oracle(qh, oracle, gpu):
    import torch
    rng = np.random.default_rng(11)
    cases = [
        (0.7, 20, 0.8, 0.0, 1.1, 0), (1.0, 55, 1.0, 0.0, 1.0, 0), (0.3, 1, 0.8, 0.0, 1.1, 0),
        (1.5, 256, 0.95, 0.01, 0.8, 7), (0.7, 40, 0.5, 0.05, 1.3, 16), (0.0, 20, 0.8, 0.0, 1.0, 0),
        (0.0, 0, 1.0, 0.0, 1.7, 5), (0.9, 0, 0.9, 0.0, 1.1, 0),
    ]
    for i, t in enumerate(cases):
        n = 200 if t[1] == 0 and t[0] > 0 else 3000  # top-k disabled: every id survives (at most 256 here)
        n_valid = n - int(rng.integers(0, 20))
        logits = (rng.normal(0.0, 2.5, n) * rng.choice([0.5, 2.0])).astype(np.float32)
        hist = rng.integers(-2, n + 3, int(rng.integers(0, 60))).astype(np.int32)
        _draws(qh, oracle, torch.from_numpy(logits).to(gpu), n_valid, hist, t, 1000 + i, 3)


def test_sample_full_vocab_pool_overflow(qh, oracle, gpu):
    """151936 candidates: the per-wave bounds leave more than the LDS pool holds, so the top-k comes from k rounds of
    a block maximum."""
    import torch
    rng = np.random.default_rng(12)
    logits = rng.normal(0.0, 3.0, 151936).astype(np.float32)
    hist = rng.integers(0, 151936, 700).astype(np.int32)
    _draws(qh, oracle, torch.from_numpy(logits).to(gpu), 151936, hist, (0.7, 20, 0.8, 0.0, 1.1, 0), 5, 4)


@pytest.mark.parametrize("t", [(0.7, 20, 0.8, 0.0, 1.1, 0), (0.0, 20, 0.8, 0.0, 1.2, 0), (1.2, 55, 0.9, 0.0, 1.1, 9),
                               (1.0, 64, 0.95, 0.0, 1.1, 0), (1.3, 256, 0.99, 0.0, 1.05, 0)])
def test_sample_over_shortlist_rows(qh, oracle, synth, gpu, t):
    """Candidates from the Exact Shortlist Head's row list (every other logit is -inf), with the history as must ids
    of the head query, as the decoder runs it."""
    import torch
    V, D = 6007, 896
    head8, head4, err = synth.shortlist_head(41, V, D)
    h8 = qh.DeviceTensor.upload(head8, 2, V, D)
    h4 = qh.DeviceTensor.upload(head4, 3, V, D)
    he = qh.DeviceTensor.upload(err.view(np.uint8), 1, V, D // 32)
    k = 1 if t[0] <= 0 else t[1]
    sl = qh.ShortlistHead(h8, h4, he, top_k=k)
    rng = np.random.default_rng(13)
    x = synth.activations(77, 3, D, scale=0.5)
    xq, xd = qh.quantize_q8(torch.from_numpy(x).to(gpu))
    for r in range(3):
        hist = rng.integers(0, V, 300).astype(np.int32)
        sl(xq[r], xd[r], must=torch.tensor(hist, device=gpu))
        _draws(qh, oracle, sl.logits, V, hist, t, 7 + r, 1, head=sl)


@pytest.mark.parametrize("V", [3000, 40000, 151936])
def test_sample_any_topk_equals_oracle(qh, oracle, gpu, V):
    """top_k 0 (every id below n_valid a survivor) and top_k above 256: qh_sample_ws's sorted path."""
    import torch
    rng = np.random.default_rng(V)
    cases = [
        (0.7, 0, 0.8, 0.0, 1.1, 0), (1.0, 0, 1.0, 0.0, 1.0, 0), (0.9, 300, 0.95, 0.05, 1.3, 16),
        (1.5, 1000, 0.999, 0.0, 1.1, 0), (2.0, 0, 1.0, 0.001, 1.0, 0), (0.5, 257, 0.9, 0.0, 0.8, 7),
        (3.0, 0, 0.99, 0.0, 1.05, 40), (0.0, 0, 1.0, 0.0, 1.3, 0),
    ]
    ws = qh.sample_workspace(V)
    for i, t in enumerate(cases):
        n_valid = V - int(rng.integers(0, 20))
        logits = (rng.normal(0.0, 2.5, V) * rng.choice([0.3, 1.0, 3.0])).astype(np.float32)
        logits[rng.integers(0, V, 40)] = logits[int(rng.integers(0, V))]  # equal logits
        hist = rng.integers(-2, V + 3, int(rng.integers(0, 600))).astype(np.int32)
        _draws(qh, oracle, torch.from_numpy(logits).to(gpu), n_valid, hist, t, 2000 + i, 3, ws=ws)


def test_sample_any_topk_needs_workspace(qh, gpu):
    import torch
    logits = torch.zeros(5000, device=gpu)
    st = _state_dev(1, gpu)
    with pytest.raises(qh.QHError):
        qh.sample(logits, qh.qh_sampler_params(0.7, 0, 0.9, 0.0, 1.0, 0), st)
    with pytest.raises(qh.QHError):  # too small
        qh.sample(logits, qh.qh_sampler_params(0.7, 300, 0.9, 0.0, 1.0, 0), st, ws=qh.sample_workspace(2000))


@pytest.mark.parametrize("t", [(0.7, 0, 0.8, 0.0, 1.1, 0), (1.3, 1000, 0.99, 0.01, 1.1, 9), (2.0, 0, 1.0, 0.0, 1.0, 0)])
def test_sample_any_topk_over_shortlist_rows(qh, oracle, synth, gpu, t):
    """The sorted path over the head's row list: the candidates are the listed rows (every other logit is -inf)."""
    import torch
    V, D = 6007, 896
    head8, head4, err = synth.shortlist_head(43, V, D)
    h8 = qh.DeviceTensor.upload(head8, 2, V, D)
    h4 = qh.DeviceTensor.upload(head4, 3, V, D)
    he = qh.DeviceTensor.upload(err.view(np.uint8), 1, V, D // 32)
    sl = qh.ShortlistHead(h8, h4, he, top_k=200)
    rng = np.random.default_rng(14)
    x = synth.activations(78, 3, D, scale=0.5)
    xq, xd = qh.quantize_q8(torch.from_numpy(x).to(gpu))
    ws = qh.sample_workspace(V)
    for r in range(3):
        hist = rng.integers(0, V, 300).astype(np.int32)
        sl(xq[r], xd[r], must=torch.tensor(hist, device=gpu))
        _draws(qh, oracle, sl.logits, V, hist, t, 9 + r, 1, head=sl, ws=ws)


FLOWS = {
    "chat_defaults": ((0.7, 20, 0.8, 0.0, 1.1, 0), (0.7, 20, 0.8, 0.0, 1.1, 0), 0x51A7C0DE),
    "chat_window_minp": ((0.9, 40, 0.95, 0.02, 1.3, 12), (0.9, 40, 0.95, 0.02, 1.3, 12), 77),
    "gen_topk20_greedy": ((0.7, 20, 0.8, 0.0, 1.1, 0), None, 1),
    "greedy_penalty": ((0.0, 20, 0.8, 0.0, 1.5, 0), (0.0, 20, 0.8, 0.0, 1.5, 0), 3),
    "chat_topk64": ((0.8, 64, 0.95, 0.0, 1.1, 0), (0.8, 64, 0.95, 0.0, 1.1, 0), 19),
    "chat_topk256": ((1.1, 256, 0.98, 0.0, 1.1, 0), (1.1, 256, 0.98, 0.0, 1.1, 0), 23),
    "gen_topk128_greedy": ((0.7, 128, 0.8, 0.0, 1.1, 0), None, 1),
    "chat_topk0": ((0.8, 0, 0.95, 0.0, 1.1, 0), (0.8, 0, 0.95, 0.0, 1.1, 0), 29),
    "chat_topk0_minp": ((1.2, 0, 1.0, 0.02, 1.0, 0), (1.2, 0, 1.0, 0.02, 1.0, 0), 31),
}


@pytest.fixture(scope="module")
def small(qh, gpu):
    qnt = qnt_module()
    hp = qnt.HParams(vocab_size=3000, n_layers=2)
    tens = qnt.synthetic_q4mix(13, hp)
    return hp, tens, qh.Decoder(hp, tens, ctx_len=256)


def _run(dec, prompt, n_gen, q, sp, seed, graph=False):
    import torch
    dec.set_query(q)
    dec.set_sampler(sp, seed)
    dec.prefill(prompt, 0)
    dec.begin(n_gen)
    if not graph:
        for _ in range(n_gen - 1):
            dec.step()
    else:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                dec.step()
        torch.cuda.current_stream().wait_stream(s)
        for _ in range(n_gen - 1):
            g.replay()
            torch.cuda.synchronize()
    out = dec.outputs(n_gen).copy()
    dec.set_query(None)
    dec.set_sampler(None)
    return out


@pytest.mark.parametrize("flow", sorted(FLOWS))
def test_decoder_sampling_flows_equal_oracle_session(qh, oracle, small, flow):
    hp, tens, dec = small
    tq, ts, seed = FLOWS[flow]
    q = qh.qh_sampler_params(*tq)
    sp = qh.qh_sampler_params(*ts) if ts is not None else None
    prompt = np.random.default_rng(17).integers(0, hp.vocab_size, 45).astype(np.int32)
    prompt[5:25] = prompt[:20]
    n_gen = 30
    orc = oracle_decoder(oracle, hp, tens, ctx_len=256)
    want, _ = oracle_session(oracle, orc, prompt, n_gen, oracle_mod.SamplerParams(*tq),
                             oracle_mod.SamplerParams(*ts) if ts is not None else None, seed, hp.vocab_size)
    got = _run(dec, prompt, n_gen, q, sp, seed)
    assert got.tolist() == want
    assert dec.history().tolist() == prompt.tolist() + want
    if flow == "chat_defaults":  # the same stream from one captured step replayed
        assert _run(dec, prompt, n_gen, q, sp, seed, graph=True).tolist() == want


def test_decoder_topk_above_head_limit(qh, oracle, small):
    """top_k above the shortlist head's limit: refused on a model with the head tensors; on one without them (f32
    matrices, the full head every step) the sorted sampler path draws the oracle session's stream."""
    _, _, dec = small
    with pytest.raises(qh.QHError):
        dec.set_query(qh.qh_sampler_params(0.7, 300, 0.9, 0.0, 1.1, 0))
    qnt = qnt_module()
    hp = qnt.HParams(vocab_size=1024, dim=256, n_layers=2, n_heads=4, n_kv_heads=1, head_dim=64, ffn_dim=512)
    tens = qnt.synthetic_dense(81, hp, 0)
    dense = qh.Decoder(hp, tens, ctx_len=128)
    orc = oracle_decoder(oracle, hp, tens, ctx_len=128)
    prompt = np.random.default_rng(18).integers(0, hp.vocab_size, 37).astype(np.int32)
    for t, seed in (((0.9, 300, 0.97, 0.0, 1.1, 0), 41), ((1.4, 0, 1.0, 0.01, 1.2, 8), 43)):
        want, _ = oracle_session(oracle, orc, prompt, 12, oracle_mod.SamplerParams(*t), oracle_mod.SamplerParams(*t),
                                 seed, hp.vocab_size)
        got = _run(dense, prompt, 12, qh.qh_sampler_params(*t), qh.qh_sampler_params(*t), seed)
        assert got.tolist() == want, t
    dense.close()


@pytest.fixture(scope="module")
def q4mix_sampled(qh, gpu):
    qnt = qnt_module()
    g = np.load(os.path.join(GOLDEN, "e2e_sampled.npz"), allow_pickle=False)
    hp = qnt.HParams()
    return qh.Decoder(hp, qnt.synthetic_q4mix(int(g["seed"]), hp), ctx_len=4096), g


@pytest.mark.parametrize("flow", ["chat", "gen"])
def test_decoder_q4mix_sampled_stream_equals_reference(qh, q4mix_sampled, flow):
    dec, g = q4mix_sampled
    chat = qh.sampler_params()
    q = chat if flow == "chat" else qh.sampler_params(top_k=20, repeat_penalty=1.1)
    dec.set_query(q)
    dec.set_sampler(chat if flow == "chat" else None, int(g["sampler_seed"]))
    want, rows = g[flow + "_out"], g[flow + "_rows"]
    n = len(want)
    dec.prefill(g["prompt"], 0)
    assert dec.stats()["n_rows"] == int(rows[0])
    dec.begin(n)
    for s in range(1, n):
        dec.step()
        assert dec.stats()["n_rows"] == int(rows[s]), s
    out = dec.outputs(n)
    dec.set_query(None)
    dec.set_sampler(None)
    assert (out == want).all(), np.nonzero(out != want)[0][:5]
