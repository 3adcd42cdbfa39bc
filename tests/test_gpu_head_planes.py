"""GPU parity of the nibble-plane shortlist head (qh_head_planes, qh_shortlist_planes) against the oracle.

The device layout must equal the oracle's byte for byte; coarse scores, upper bounds, the rescored rows and their
logits, tau and the greedy token must equal the oracle's (qo_shortlist_planes), and every rescored logit and the
top-1 the full Q8_0 head's (the exact rows are rebuilt from both planes).
"""
import numpy as np
import pytest

from conftest import bits

pytestmark = pytest.mark.gpu


def _dev(a, gpu):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(gpu)


def _planes_head(qh, oracle, head8, V, D):
    h8 = qh.DeviceTensor.upload(head8, qh.Q8_0, V, D)
    pl = qh.head_planes(h8)
    assert np.array_equal(pl.buf.cpu().numpy(), oracle.head_planes(head8, V, D)), "plane layout"
    return h8, pl


def _check(qh, oracle, planes_np, sl, xq, xd, V, D, top_k, n_valid=0, must=None):
    import torch
    must_t = None if must is None else torch.tensor(must, dtype=torch.int32, device=xq.device)
    sl(xq, xd, n_valid=n_valid, must=must_t)
    st = sl.stats()
    o = oracle.shortlist_planes(planes_np, V, D, xq.cpu().numpy(), xd.cpu().numpy(), top_k=top_k, n_valid=n_valid,
                                must=must)
    assert not st["seed_tie"] and not o["seed_tie"]
    assert (bits(sl.coarse.cpu().numpy()) == bits(o["coarse"])).all(), "coarse"
    assert (bits(sl.upper.cpu().numpy()) == bits(o["upper"])).all(), "upper"
    assert st["n_rows"] == o["n_rows"] and st["n_seeds"] == o["n_seeds"]
    rows = sl.rows.cpu().numpy()[: st["n_rows"]]
    assert sorted(rows.tolist()) == sorted(o["rows"].tolist())
    assert rows[: st["n_seeds"]].tolist() == o["rows"][: o["n_seeds"]].tolist(), "seed order"
    nm = st["n_must"]
    if nm:
        assert rows[len(rows) - nm:].tolist() == o["rows"][len(o["rows"]) - nm:].tolist(), "must ids last"
    assert (bits(sl.logits.cpu().numpy()) == bits(o["logits"])).all(), "logits"
    assert np.float32(st["tau"]).tobytes() == np.float32(o["tau"]).tobytes()
    nv = n_valid if 0 < n_valid < V else V
    assert st["top1"] == oracle.argmax(o["logits"], nv)
    return st, o


@pytest.mark.parametrize("top_k", [1, 20, 64, 256])
def test_planes_small_vocab(qh, oracle, synth, gpu, top_k):
    V, D = 6007, 896
    head8 = synth.q8_tensor(41, V, D)
    h8, pl = _planes_head(qh, oracle, head8, V, D)
    planes_np = pl.buf.cpu().numpy()
    sl = qh.ShortlistHead(pl, None, None, top_k=top_k)
    x = synth.activations(43, 6, D, scale=0.5)
    xq, xd = qh.quantize_q8(_dev(x, gpu))
    for t in range(4):
        st, o = _check(qh, oracle, planes_np, sl, xq[t], xd[t], V, D, top_k)
        full = qh.matvec_q(h8, xq[t], xd[t]).cpu().numpy()
        rows = o["rows"]
        assert (bits(o["logits"][rows]) == bits(full[rows])).all(), "rescored logits = the full Q8_0 head's"
        assert st["top1"] == oracle.argmax(full, V)
    must = [5, 17, 5, 6000, -3, 4000, 123, 17]
    _check(qh, oracle, planes_np, sl, xq[4], xd[4], V, D, top_k, n_valid=5000, must=must)
    _check(qh, oracle, planes_np, sl, xq[5], xd[5], V, D, top_k, n_valid=5000, must=must)


def test_planes_full_vocab(qh, oracle, synth, gpu):
    """The benchmark head's shape (151,936 x 896), top_k 1 and 20 with a history-like must list."""
    V, D = 151936, 896
    head8 = synth.q8_tensor(47, V, D)
    h8, pl = _planes_head(qh, oracle, head8, V, D)
    planes_np = pl.buf.cpu().numpy()
    x = synth.activations(53, 4, D, scale=0.5)
    xq, xd = qh.quantize_q8(_dev(x, gpu))
    sl = qh.ShortlistHead(pl, None, None, top_k=1)
    for t in range(3):
        print(f"planes full vocab, top_k 1, vector {t}", flush=True)
        st, o = _check(qh, oracle, planes_np, sl, xq[t], xd[t], V, D, 1)
        full = qh.matvec_q(h8, xq[t], xd[t])
        assert st["top1"] == int(qh.argmax(full).item())
        assert np.float32(st["top1_logit"]).tobytes() == full[st["top1"]].cpu().numpy().tobytes()
        assert 0 < st["n_rows"] < V // 20
    sl20 = qh.ShortlistHead(pl, None, None, top_k=20)
    must = np.random.default_rng(61).integers(0, V, 500).tolist()
    print("planes full vocab, top_k 20 with must ids", flush=True)
    _check(qh, oracle, planes_np, sl20, xq[3], xd[3], V, D, 20, must=must)


def test_planes_sweep_equals_full_head(qh, synth, gpu):
    """1,024 hidden states N(0,1)*0.5 on the 151,936-row head: the nibble-plane head's greedy token and its logit are
    the full Q8_0 head's first argmax, every time."""
    import torch
    V, D = 151936, 896
    head8 = synth.q8_tensor(47, V, D)
    h8 = qh.DeviceTensor.upload(head8, qh.Q8_0, V, D)
    pl = qh.head_planes(h8)
    sl = qh.ShortlistHead(pl, None, None, top_k=1)
    am = qh.Argmax(V)
    x = synth.activations(502, 1024, D, scale=0.5)
    xq, xd = qh.quantize_q8(_dev(x, gpu))
    full = torch.empty(V, dtype=torch.float32, device=gpu)
    tops = torch.empty(1024, dtype=torch.int32, device=gpu)
    logit = torch.empty(1024, dtype=torch.float32, device=gpu)
    want = torch.empty(1024, dtype=torch.int32, device=gpu)
    want_logit = torch.empty(1024, dtype=torch.float32, device=gpu)
    n_rows = []
    for t in range(1024):
        sl(xq[t], xd[t])
        tops[t] = sl.stats_dev[0]
        logit[t] = sl.stats_dev[7:8].view(torch.float32)[0]
        n_rows.append(sl.stats_dev[1].clone())
        qh.matvec_q(h8, xq[t], xd[t], out=full)
        want[t] = am(full)
        want_logit[t] = full[want[t].long()]
    assert torch.equal(tops, want)
    assert torch.equal(logit.view(torch.int32), want_logit.view(torch.int32))
    rows = torch.stack(n_rows).cpu().numpy()
    print(f"planes sweep: rescored rows mean {rows.mean():.1f}, max {rows.max()}", flush=True)
    assert rows.max() < V // 20


def test_matvec_planes_equals_q8(qh, synth, gpu):
    """qh_matvec_q over the plane layout equals the Q8_0 GEMV of the same values bit for bit, row ranges included."""
    import torch
    V, D = 5003, 896
    head8 = synth.q8_tensor(57, V, D)
    h8 = qh.DeviceTensor.upload(head8, qh.Q8_0, V, D)
    pl = qh.head_planes(h8)
    x = synth.activations(58, 2, D, scale=0.5)
    xq, xd = qh.quantize_q8(_dev(x, gpu))
    for t in range(2):
        want = qh.matvec_q(h8, xq[t], xd[t]).cpu().numpy()
        got = qh.matvec_q(pl, xq[t], xd[t]).cpu().numpy()
        assert (bits(got) == bits(want)).all()
        part = torch.full((V,), 7.0, device=gpu)
        qh.matvec_q(pl, xq[t], xd[t], out=part, r0=300, r1=4100)
        p = part.cpu().numpy()
        assert (bits(p[300:4100]) == bits(want[300:4100])).all() and (p[:300] == 7).all() and (p[4100:] == 7).all()


def test_decoder_planes_equals_oracle(qh, oracle, gpu):
    """A decoder whose tied embedding / LM head is stored as nibble planes (no head_q4 / head_err uploaded): the
    embedding rows come from the planes, shortlist steps equal the oracle's nibble-plane head on the same hidden
    state, full-head steps (the plane GEMV) equal the oracle's full 8-bit head, every hidden state bit for bit."""
    from decoder_util import oracle_decoder, qnt_module
    qnt = qnt_module()
    hp = qnt.HParams(vocab_size=3072, n_layers=3)
    tens = qnt.synthetic_q4mix(23, hp)
    V, D = hp.vocab_size, hp.dim
    planes_np = oracle.head_planes(np.asarray(tens["model.embed_tokens.weight"].data), V, D)
    ctx = 512
    orc = oracle_decoder(oracle, hp, tens, ctx_len=ctx)
    dec = qh.Decoder(hp, tens, ctx_len=ctx, head_planes=True)

    def check_shortlist(tag):
        hq, hd = dec.hq()
        o = oracle.shortlist_planes(planes_np, V, D, hq, hd, top_k=1)
        assert dec.stats()["n_rows"] == o["n_rows"], tag
        assert (bits(dec.logits()) == bits(o["logits"])).all(), tag
        return oracle.argmax(o["logits"], V)

    ids = np.random.default_rng(5).integers(0, V, 77).astype(np.int32)
    r = orc.forward_batch(ids, 0, top_k=0)
    dec.prefill(ids, 0, top_k=1)
    assert (bits(dec.hidden()) == bits(r["hidden"])).all()
    tok = check_shortlist("prefill")
    assert tok == oracle.argmax(r["logits"])
    dec.begin(16, top_k=1)
    pos = len(ids)
    for step in range(8):
        top_k = 0 if step % 3 == 2 else 1
        r = orc.forward(tok, pos, top_k=0)
        dec.step(top_k=top_k)
        assert (bits(dec.hidden()) == bits(r["hidden"])).all(), step
        if top_k:
            assert check_shortlist(step) == oracle.argmax(r["logits"]), step
        else:
            assert (bits(dec.logits()) == bits(r["logits"])).all(), step
            assert dec.top1_full() == oracle.argmax(r["logits"]), step
        tok = oracle.argmax(r["logits"])
        pos += 1


def test_decoder_planes_q4mix_stream_equals_reference(qh, oracle, gpu):
    """The benchmark model with its tied head as nibble planes: the 256 greedy tokens after the 512-token prompt equal
    the reference's gen stream, with each forward's chosen logit and final-state digest (tests/golden/e2e_q4mix.npz);
    the rescored rows equal the oracle's nibble-plane head at every 64th forward."""
    import os
    from conftest import GOLDEN
    from decoder_util import qnt_module
    from test_gpu_decoder import state_digest
    qnt = qnt_module()
    g = np.load(os.path.join(GOLDEN, "e2e_q4mix.npz"), allow_pickle=False)
    hp = qnt.HParams()
    tens = qnt.synthetic_q4mix(int(g["seed"]), hp)
    V, D = hp.vocab_size, hp.dim
    planes_np = oracle.head_planes(np.asarray(tens["model.embed_tokens.weight"].data), V, D)
    dec = qh.Decoder(hp, tens, ctx_len=4096, head_planes=True)
    del tens
    n_gen = len(g["out"])
    dec.prefill(g["prompt"], 0, top_k=1)
    dec.begin(n_gen + 1)
    tops, digs = [], []
    for s in range(n_gen + 1):
        st = dec.stats()
        tops.append(st["top1_logit"])
        digs.append(state_digest(dec.hidden(), *dec.hq()))
        if s % 64 == 0:
            hq, hd = dec.hq()
            o = oracle.shortlist_planes(planes_np, V, D, hq, hd, top_k=1)
            assert st["n_rows"] == o["n_rows"], s
        if s < n_gen:
            dec.step(top_k=1)
    out = dec.outputs(n_gen)
    assert (out == g["out"]).all()
    assert (np.array(digs) == g["state_digests"]).all()
    assert (bits(np.array(tops[:n_gen], np.float32)) == bits(g["top_logit"])).all()


@pytest.mark.parametrize("flow", ["chat", "gen"])
def test_decoder_planes_sampled_stream_equals_reference(qh, gpu, flow):
    """The benchmark model's sampling flows with the nibble-plane head: top-k 20 queries with the token history as
    must ids and the reference Sampler's draws (chat: temperature 0.7, top-p 0.8, penalty 1.1; gen: greedy with
    penalty). The head rescores other rows than the Q4_0 copy's, but every row the sampler can keep (the top-k and
    the must ids) is exact in both, so the stream equals the reference Session's (tests/golden/e2e_sampled.npz)."""
    import os
    from conftest import GOLDEN
    from decoder_util import qnt_module
    qnt = qnt_module()
    g = np.load(os.path.join(GOLDEN, "e2e_sampled.npz"), allow_pickle=False)
    hp = qnt.HParams()
    dec = qh.Decoder(hp, qnt.synthetic_q4mix(int(g["seed"]), hp), ctx_len=4096, head_planes=True)
    chat = qh.sampler_params()
    q = chat if flow == "chat" else qh.sampler_params(top_k=20, repeat_penalty=1.1)
    dec.set_query(q)
    dec.set_sampler(chat if flow == "chat" else None, int(g["sampler_seed"]))
    want = g[flow + "_out"]
    n = len(want)
    dec.prefill(g["prompt"], 0)
    dec.begin(n)
    for _ in range(1, n):
        dec.step()
    out = dec.outputs(n)
    dec.close()
    assert (out == want).all(), np.nonzero(out != want)[0][:5]
