"""GPU parity of the decoder (qh_decoder_*), through the C-ABI.

* small synthetic model (2 layers, vocab 4096): after the batched prefill and after every greedy decode step, the final
  normed hidden state, its int8 quantization, the 8-bit head rows and the token equal what the reference engine wrote
  (tests/golden/e2e_small.npz), bit for bit;
* another seed, 3 layers, a prompt longer than one 32-token chunk, shortlist and full-head steps: hidden states and
  logits equal the oracle's decoder restatement, bit for bit;
* the benchmark model (24 layers, vocab 151936), written to a .qnt file and read back by qnt.load_model: 512-token
  prompt, 256 greedy tokens equal the reference's `gen` stream (tests/golden/e2e_q4mix.npz), with each step's head
  rows, the exact logit of the chosen token and a digest of the final normed hidden state and its quantization;
* a chat's second turn: a prefill at pos0 > 0 (after a prefill, and after decode steps) equals the oracle's, cache and
  history included;
* one decode step captured in a HIP graph and replayed gives the same stream as eager steps;
* head_dim 128, a context longer than one LDS stage of V rows, and the one-launch-per-operation path
  (QH_DECODER_FUSE=0) all equal the oracle bit for bit;
* a step past the context and an out-of-range prompt token raise the status bits and touch nothing out of bounds.
"""
import os

import numpy as np
import pytest

from conftest import GOLDEN, bits
from decoder_util import oracle_decoder, qnt_module

pytestmark = pytest.mark.gpu


def _golden(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def test_decoder_small_model_matches_reference_states(qh, gpu):
    qnt = qnt_module()
    g = _golden("e2e_small.npz")
    hp = qnt.HParams(vocab_size=int(g["vocab"]), n_layers=int(g["n_layers"]))
    dec = qh.Decoder(hp, qnt.synthetic_q4mix(int(g["seed"]), hp), ctx_len=256)
    dec.prefill(g["prompt"], 0, top_k=1)
    n_gen = len(g["out"])
    dec.begin(n_gen + 1)
    for s in range(n_gen + 1):
        st = dec.stats()
        assert st["n_rows"] == int(g["head_rows"][s]), s
        assert (bits(dec.hidden()) == bits(g["hidden"][s])).all(), f"hidden state after step {s}"
        q, d = dec.hq()
        assert (q == g["hq"][s]).all() and (bits(d) == bits(g["hd"][s])).all(), s
        if s == n_gen:
            break
        dec.step(top_k=1)
    assert (dec.outputs(n_gen) == g["out"]).all()


def _steps_vs_oracle(oracle, orc, dec, ids, n_steps, full_every=0, shortlist=True):
    """Prefill `ids` on both, then n_steps greedy steps; every hidden state, logit and row count bit-equal (without
    shortlist tensors every head call is the full head, whose greedy token is compared instead)."""
    r = orc.forward_batch(ids, 0, top_k=1)
    dec.prefill(ids, 0, top_k=1)
    assert (bits(dec.hidden()) == bits(r["hidden"])).all(), "hidden state after the prefill"
    assert (bits(dec.logits()) == bits(r["logits"])).all(), "logits after the prefill"
    if shortlist:
        assert dec.stats()["n_rows"] == r["rows"]
    else:
        assert r["rows"] == len(r["logits"]) and dec.top1_full() == oracle.argmax(r["logits"])
    dec.begin(n_steps + 1, top_k=1)
    pos = len(ids)
    tok = int(np.argmax(r["logits"]))
    for step in range(n_steps):
        top_k = 0 if full_every and step % full_every == full_every - 1 else 1
        r = orc.forward(tok, pos, top_k=top_k)
        dec.step(top_k=top_k)
        assert (bits(dec.hidden()) == bits(r["hidden"])).all(), f"hidden state, step {step}"
        assert (bits(dec.logits()) == bits(r["logits"])).all(), f"logits, step {step}"
        if top_k and shortlist:
            assert dec.stats()["n_rows"] == r["rows"], step
        else:
            assert dec.top1_full() == oracle.argmax(r["logits"]), step
        tok = oracle.argmax(r["logits"])
        pos += 1
    assert dec.status() == 0
    return dec.outputs(n_steps + 1)


def _narrow_hp(qnt, **kw):
    base = dict(vocab_size=1024, dim=256, n_layers=2, n_heads=4, n_kv_heads=1, head_dim=64, ffn_dim=512)
    base.update(kw)
    return qnt.HParams(**base)


def test_decoder_head_dim_128_equals_oracle(qh, oracle, gpu):
    qnt = qnt_module()
    hp = _narrow_hp(qnt, n_heads=2, n_kv_heads=1, head_dim=128)
    tens = qnt.synthetic_q4mix(31, hp)
    orc = oracle_decoder(oracle, hp, tens, ctx_len=256)
    dec = qh.Decoder(hp, tens, ctx_len=256)
    ids = np.random.default_rng(8).integers(0, hp.vocab_size, 45).astype(np.int32)
    _steps_vs_oracle(oracle, orc, dec, ids, 6, full_every=3)


@pytest.mark.parametrize("dim,ffn", [(1280, 1024), (2560, 512)])
def test_decoder_wide_rows_equal_oracle(qh, oracle, gpu, dim, ffn):
    """Rows of more than two 16-block chunks: the prefill's fused gate / up / SwiGLU launch in its chunk loop (40 and
    80 blocks a row), the staged matmul's longer rows and the decode GEMVs at those widths; 45 prompt tokens end in a
    partial token tile."""
    qnt = qnt_module()
    hp = _narrow_hp(qnt, dim=dim, n_heads=dim // 64, n_kv_heads=dim // 320, ffn_dim=ffn, n_layers=1)
    tens = qnt.synthetic_q4mix(33, hp)
    orc = oracle_decoder(oracle, hp, tens, ctx_len=128)
    dec = qh.Decoder(hp, tens, ctx_len=128)
    ids = np.random.default_rng(9).integers(0, hp.vocab_size, 45).astype(np.int32)
    _steps_vs_oracle(oracle, orc, dec, ids, 3, full_every=2)


def test_decoder_context_beyond_one_v_stage(qh, oracle, gpu):
    # head_dim 64 stages 768 V rows in LDS at a time: a 1000-token prompt puts prefill chunks and decode steps past it
    qnt = qnt_module()
    hp = _narrow_hp(qnt)
    tens = qnt.synthetic_q4mix(37, hp)
    orc = oracle_decoder(oracle, hp, tens, ctx_len=1100)
    dec = qh.Decoder(hp, tens, ctx_len=1100)
    ids = np.random.default_rng(12).integers(0, hp.vocab_size, 1000).astype(np.int32)
    _steps_vs_oracle(oracle, orc, dec, ids, 6)


@pytest.mark.parametrize("n_prompt,n_steps", [(1020, 580), (2290, 30)])
def test_decoder_decode_past_1024_positions(qh, oracle, gpu, n_prompt, n_steps):
    """Decode steps across positions 1024, 1536, 2048 and 2304: the decode attention scores positions beyond its
    1024 threads in a loop (the token's own row by thread pos % 1024 there), and the V rows pass through three and
    four LDS stages of 768. Every step's hidden state and logits equal the oracle's bit for bit."""
    qnt = qnt_module()
    hp = _narrow_hp(qnt)
    tens = qnt.synthetic_q4mix(39, hp)
    orc = oracle_decoder(oracle, hp, tens, ctx_len=2400)
    dec = qh.Decoder(hp, tens, ctx_len=2400)
    ids = np.random.default_rng(15).integers(0, hp.vocab_size, n_prompt).astype(np.int32)
    _steps_vs_oracle(oracle, orc, dec, ids, n_steps)


def test_decoder_fused_equals_one_launch_per_op(qh, oracle, gpu, monkeypatch):
    qnt = qnt_module()
    hp = qnt.HParams(vocab_size=4096, n_layers=2)
    tens = qnt.synthetic_q4mix(41, hp)
    ids = np.random.default_rng(13).integers(0, hp.vocab_size, 70).astype(np.int32)
    outs = []
    for fuse in ("1", "0"):
        monkeypatch.setenv("QH_DECODER_FUSE", fuse)
        orc = oracle_decoder(oracle, hp, tens, ctx_len=256)
        dec = qh.Decoder(hp, tens, ctx_len=256)
        outs.append(_steps_vs_oracle(oracle, orc, dec, ids, 10, full_every=4))
        dec.close()
    assert (outs[0] == outs[1]).all()


def test_decoder_status_past_context_and_bad_token(qh, gpu):
    qnt = qnt_module()
    hp = _narrow_hp(qnt)
    tens = qnt.synthetic_q4mix(43, hp)
    ids = np.random.default_rng(14).integers(0, hp.vocab_size, 40).astype(np.int32)
    wide = qh.Decoder(hp, tens, ctx_len=128)
    wide.prefill(ids, 0, top_k=1)
    wide.begin(13)
    for _ in range(12):
        wide.step(top_k=1)
    dec = qh.Decoder(hp, tens, ctx_len=48)
    dec.prefill(ids, 0, top_k=1)
    dec.begin(13)
    for s in range(12):
        dec.step(top_k=1)
        assert dec.status() == (0 if 40 + s < 48 else 1), s
    assert dec.position() == 52
    # the steps inside the context are the same as with room to spare
    assert (dec.outputs(9) == wide.outputs(9)).all()
    bad = ids.copy()
    bad[5] = hp.vocab_size
    dec.prefill(bad, 0, top_k=1)
    assert dec.status() == 2
    bad[5] = -1
    dec.prefill(bad, 0, top_k=1)
    assert dec.status() == 2
    dec.prefill(ids, 0, top_k=1)
    assert dec.status() == 0


def test_decoder_equals_oracle_long_prompt_and_full_head(qh, oracle, gpu):
    qnt = qnt_module()
    hp = qnt.HParams(vocab_size=3072, n_layers=3)
    tens = qnt.synthetic_q4mix(23, hp)
    ctx = 512
    orc = oracle_decoder(oracle, hp, tens, ctx_len=ctx)
    dec = qh.Decoder(hp, tens, ctx_len=ctx)
    ids = np.random.default_rng(5).integers(0, hp.vocab_size, 77).astype(np.int32)
    r = orc.forward_batch(ids, 0, top_k=1)
    dec.prefill(ids, 0, top_k=1)
    assert (bits(dec.hidden()) == bits(r["hidden"])).all()
    assert (bits(dec.logits()) == bits(r["logits"])).all()
    assert dec.stats()["n_rows"] == r["rows"]
    dec.begin(16, top_k=1)
    pos = len(ids)
    tok = int(np.argmax(r["logits"]))
    for step in range(8):
        top_k = 0 if step % 3 == 2 else 1
        r = orc.forward(tok, pos, top_k=top_k)
        dec.step(top_k=top_k)
        assert (bits(dec.hidden()) == bits(r["hidden"])).all(), step
        if top_k:
            assert (bits(dec.logits()) == bits(r["logits"])).all(), step
            assert dec.stats()["n_rows"] == r["rows"], step
        else:
            assert (bits(dec.logits()) == bits(r["logits"])).all(), step
            assert dec.top1_full() == oracle.argmax(r["logits"]), step
        tok = oracle.argmax(r["logits"])
        pos += 1
    assert dec.outputs(9)[1:].tolist() == [int(x) for x in dec.outputs(9)[1:]]


def state_digest(hidden, hq, hd):
    """The golden's per-forward fingerprint (tests/golden/make_e2e_golden.py): 8 bytes of the sha256 of the final normed
    hidden state, then of its int8 quantization and block scales."""
    import hashlib
    h1 = hashlib.sha256(np.ascontiguousarray(hidden, np.float32).tobytes()).digest()[:8]
    h2 = hashlib.sha256(np.ascontiguousarray(hq, np.int8).tobytes() +
                        np.ascontiguousarray(hd, np.float32).tobytes()).digest()[:8]
    return np.frombuffer(h1 + h2, np.uint64)


@pytest.fixture(scope="module")
def q4mix(qh, gpu, tmp_path_factory):
    """The benchmark model from a file on disk: written by qnt.write_qnt, read back by qnt.load_model (the .qnt reader
    and Model::load's checks, model_file.cpp:104-218, model.cpp:10-58), uploaded by Decoder."""
    qnt = qnt_module()
    import hashlib
    g = _golden("e2e_q4mix.npz")
    path = str(tmp_path_factory.mktemp("q4mix") / "q4mix.qnt")
    qnt.write_qnt(path, qnt.HParams(), qnt.synthetic_q4mix(int(g["seed"]), qnt.HParams()))
    hp, n_tokens, tens = qnt.load_model(path)
    want = qnt.HParams()
    assert n_tokens == hp.vocab_size and (hp.vocab_size, hp.dim, hp.n_layers, hp.max_seq) == (
        want.vocab_size, want.dim, want.n_layers, want.max_seq)
    assert np.float32(hp.norm_eps) == np.float32(want.norm_eps) and hp.rope_theta == want.rope_theta
    for name, want in zip(g["digest_names"], g["digests"]):
        got = hashlib.sha256(np.ascontiguousarray(tens[str(name)].data).view(np.uint8).tobytes()).hexdigest()
        assert got == str(want), f"{name} read from the file differs from the one the golden stream was made with"
    dec = qh.Decoder(hp, tens, ctx_len=4096)
    del tens
    return dec, g


def test_decoder_q4mix_stream_equals_reference(qh, q4mix):
    """256 greedy tokens after the 512-token prompt equal the reference's gen stream, with each forward's head rows,
    chosen logit and final-state digest."""
    dec, g = q4mix
    n_gen = len(g["out"])
    dec.prefill(g["prompt"], 0, top_k=1)
    dec.begin(n_gen + 1)
    rows, tops, digs = [], [], []
    for s in range(n_gen):
        st = dec.stats()
        rows.append(st["n_rows"])
        tops.append(st["top1_logit"])
        digs.append(state_digest(dec.hidden(), *dec.hq()))
        dec.step(top_k=1)
    digs.append(state_digest(dec.hidden(), *dec.hq()))
    out = dec.outputs(n_gen)
    first = int(np.nonzero(out != g["out"])[0][0]) if (out != g["out"]).any() else -1
    assert first < 0, f"token stream differs from step {first}: {out[first:first + 4]} vs {g['out'][first:first + 4]}"
    digs = np.array(digs)
    bad = np.nonzero((digs != g["state_digests"]).any(axis=1))[0]
    assert bad.size == 0, f"final normed state differs after forward {bad[:4]} (0 = the prefill)"
    assert rows == g["head_rows"].tolist()
    assert (bits(np.array(tops, np.float32)) == bits(g["top_logit"])).all()


def test_decoder_graph_replay_equals_eager(qh, q4mix):
    import torch
    dec, g = q4mix
    n = 48
    dec.prefill(g["prompt"][:300], 0, top_k=1)
    dec.begin(n + 1)
    for _ in range(n):
        dec.step(top_k=1)
    eager = dec.outputs(n + 1).copy()
    dec.prefill(g["prompt"][:300], 0, top_k=1)
    dec.begin(n + 1)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            dec.step(top_k=1)
    torch.cuda.current_stream().wait_stream(s)
    for _ in range(n):
        graph.replay()
        torch.cuda.synchronize()  # eager work of the program between replays
    assert (dec.outputs(n + 1) == eager).all()


@pytest.mark.parametrize("n_steps", [0, 3])
def test_decoder_second_turn_prefill(qh, oracle, gpu, n_steps):
    """A chat's second turn (check_batch's pos0 = 40, n = 45, engine/src/checks.cpp:148-176; session.cpp:13-31): a
    prefill at pos0 > 0 over the cache of an earlier prefill, directly and after three decode steps (pos0 = 43 starts
    inside an 8-position V block that holds decode rows). Logits, hidden state, head rows, every layer's K/V cache rows
    and the token history equal the oracle's; the batched logits also equal one-token prefills at every position."""
    qnt = qnt_module()
    hp = qnt.HParams(vocab_size=3072, n_layers=3)
    tens = qnt.synthetic_q4mix(23, hp)
    ctx = 512
    ids = np.random.default_rng(31).integers(0, hp.vocab_size, 85).astype(np.int32)
    orc = oracle_decoder(oracle, hp, tens, ctx_len=ctx)
    dec = qh.Decoder(hp, tens, ctx_len=ctx)
    r = orc.forward_batch(ids[:40], 0, top_k=1)
    dec.prefill(ids[:40], 0, top_k=1)
    assert (bits(dec.logits()) == bits(r["logits"])).all()
    hist = ids[:40].tolist()
    pos = 40
    if n_steps:
        dec.begin(n_steps + 1, top_k=1)
        hist.append(oracle.argmax(r["logits"]))
        for _ in range(n_steps):
            r = orc.forward(hist[-1], pos, top_k=1)
            dec.step(top_k=1)
            assert (bits(dec.hidden()) == bits(r["hidden"])).all()
            hist.append(oracle.argmax(r["logits"]))
            pos += 1
        assert dec.outputs(n_steps + 1).tolist() == hist[40:]
    assert dec.position() == pos
    print(f"second turn: prefill 45 tokens at pos0 {pos}", flush=True)
    r = orc.forward_batch(ids[40:85], pos, top_k=1)
    dec.prefill(ids[40:85], pos, top_k=1)
    assert (bits(dec.hidden()) == bits(r["hidden"])).all()
    assert (bits(dec.logits()) == bits(r["logits"])).all()
    assert dec.stats()["n_rows"] == r["rows"]
    assert dec.position() == pos + 45 and dec.status() == 0
    assert dec.history().tolist() == hist + ids[40:85].tolist()
    kvd = hp.n_kv_heads * hp.head_dim
    for l in range(hp.n_layers):
        gk, gv = dec.kv(l, pos + 45)
        ok, ov = orc.kv(l, pos + 45, kvd)
        assert (gk == ok).all() and (gv == ov).all(), l
    if n_steps == 0:  # check_batch: the batched logits equal the token-by-token ones (one-token prefills)
        want = dec.logits().copy()
        for p in range(85):
            dec.prefill(ids[p:p + 1], p, top_k=0)
        assert (bits(dec.logits()) == bits(orc.forward(int(ids[84]), 84, top_k=0)["logits"])).all()
        full = dec.logits()
        rows = np.isfinite(want)
        assert (bits(full[rows]) == bits(want[rows])).all()


def test_decoder_step_timed_equals_step(qh, gpu):
    """qh_decoder_step_timed runs the same step as qh_decoder_step: the same token, hidden state and logits, with one
    device time and a valid stage id per kernel (five per layer, the final norm, the head's two); with too few timing
    slots it reports QH_ERR_NOMEM and the count it needs, and the step has still run."""
    import ctypes as C
    import torch
    qnt = qnt_module()
    g = _golden("e2e_small.npz")
    hp = qnt.HParams(vocab_size=int(g["vocab"]), n_layers=int(g["n_layers"]))
    dec = qh.Decoder(hp, qnt.synthetic_q4mix(int(g["seed"]), hp), ctx_len=256)
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    L = qh.lib()

    def timed(cap):
        us = np.zeros(max(cap, 1), np.float32)
        stage = np.full(max(cap, 1), -7, np.int32)
        n = C.c_int32(-1)
        rc = L.qh_decoder_step_timed(dec.h, 1, stream, us.ctypes.data, stage.ctypes.data, cap, C.byref(n))
        return rc, n.value, us, stage

    def run(mode):
        dec.prefill(g["prompt"], 0, top_k=1)
        dec.begin(4)
        if mode == "plain":
            dec.step(top_k=1)
            dec.step(top_k=1)
            return None
        rc, n, us, stage = timed(64)
        assert rc == 0, L.qh_last_error().decode()
        rc2, n2, _, _ = timed(3)  # too few slots: refused after the step ran
        assert rc2 == qh.ERR_NOMEM and b"the step has run" in L.qh_last_error()
        assert n2 == n
        return n, us, stage

    run("plain")
    want = (dec.outputs(3).tolist(), bits(dec.hidden()), bits(dec.logits()), dec.position())
    n, us, stage = run("timed")
    got = (dec.outputs(3).tolist(), bits(dec.hidden()), bits(dec.logits()), dec.position())
    assert got[0] == want[0] and (got[1] == want[1]).all() and (got[2] == want[2]).all() and got[3] == want[3]
    assert n == 5 * hp.n_layers + 3
    ids = stage[:n].tolist()
    per_layer = [s for s in ids if s < qh.STAGE_FINAL_NORM]
    assert per_layer == [l * qh.STAGES_PER_LAYER + k for l in range(hp.n_layers) for k in range(5)]
    assert ids[5 * hp.n_layers:] == [qh.STAGE_FINAL_NORM, qh.STAGE_HEAD, qh.STAGE_HEAD]
    assert (us[:n] > 0).all() and (us[:n] < 1e5).all()
    assert dec.status() == 0
