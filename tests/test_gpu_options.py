"""GPU parity of the decoder's load-time options (Model::load, reference model.cpp:10-106), through the C-ABI:

* an untied LM head (lm_head.weight, model.cpp:16), the Hadamard-rotated down projection (FLAG_HADAMARD_DOWN,
  model.cpp:219, 424), the f32 KV cache (--kv-f32, model.cpp:96-104) and all three together, each on a 2-layer,
  vocabulary-4096 model: after the batched prefill and every greedy decode step, the final normed hidden state, its
  quantization, the head rows and the token equal what the reference engine wrote (tests/golden/e2e_options.npz),
  bit for bit; then one full-head step's logits equal the reference's (sha256) and its greedy token;
* narrower models with head_dim 64 and 128 against the oracle's decoder bit for bit, with prompts longer than one
  32-token chunk, a second prefill at pos0 > 0 (cached rows and chunk rows in one attention), contexts past one LDS
  stage of V rows, shortlist and full-head steps, and the f32 cache itself compared row for row;
* the same with one launch per operation (QH_DECODER_FUSE=0);
* unquantized weights (the exporter's --dtype f32 / f16: matvec_ref, ops_ref.cpp:8-27, and get_row, ops_ref.cpp:162-192):
  qh_matvec_ref against the oracle at the decoder's shapes and ragged row ranges; whole F32 / F16 models against the
  reference's states (e2e_options.npz) and the oracle; models mixing Q8_0, Q4_0, F32 and F16 matrices and embeddings,
  with the fused kernels on and off.
"""
import os

import numpy as np
import pytest

from conftest import GOLDEN, bits
from decoder_util import logits_sha256, option_model, oracle_decoder, qnt_module
from test_gpu_decoder import _steps_vs_oracle

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["untied", "hadamard", "kv_f32", "all", "f32", "f16"])
def test_options_match_reference_states(qh, gpu, name):
    g = np.load(os.path.join(GOLDEN, "e2e_options.npz"), allow_pickle=False)
    hp, tens, kv_f32 = option_model(g, name)
    dec = qh.Decoder(hp, tens, ctx_len=256, kv_f32=kv_f32)
    dec.prefill(g[f"{name}_prompt"], 0, top_k=1)
    n_gen = len(g[f"{name}_out"])
    dec.begin(n_gen + 2)
    dense = int(g[f"{name}_dtype"]) >= 0  # no shortlist tensors: every head call is the full head
    for s in range(n_gen + 1):
        if dense:
            assert int(g[f"{name}_head_rows"][s]) == hp.vocab_size
        else:
            assert dec.stats()["n_rows"] == int(g[f"{name}_head_rows"][s]), (name, s)
        assert (bits(dec.hidden()) == bits(g[f"{name}_hidden"][s])).all(), f"{name}: hidden state after step {s}"
        if not dense:  # an unquantized model quantizes nothing in the reference
            q, d = dec.hq()
            assert (q == g[f"{name}_hq"][s]).all() and (bits(d) == bits(g[f"{name}_hd"][s])).all(), (name, s)
        if s < n_gen:
            dec.step(top_k=1)
    out = dec.outputs(n_gen + 1)
    assert (out[:n_gen] == g[f"{name}_out"]).all()
    assert int(out[n_gen]) == int(g[f"{name}_full_token"])
    dec.step(top_k=0)  # the full head over the same hidden state path
    assert logits_sha256(dec.logits()) == str(g[f"{name}_full_logits_sha256"]), name
    assert dec.status() == 0
    dec.close()


def _narrow(qnt, **kw):
    base = dict(vocab_size=1024, dim=256, n_layers=2, n_heads=4, n_kv_heads=1, head_dim=64, ffn_dim=512)
    base.update(kw)
    return qnt.HParams(**base)


def _kv_equal(dec, orc, hp, n_pos):
    kvd = hp.n_kv_heads * hp.head_dim
    for l in range(hp.n_layers):
        k, v = dec.kv(l, n_pos)
        ok, ov = orc.kv(l, n_pos, kvd)
        assert (bits(k) == bits(ok)).all() and (bits(v) == bits(ov)).all(), f"layer {l} cache"


@pytest.mark.parametrize("head_dim,tied,flags,kv_f32,n_prompt", [
    (64, False, 1, True, 45),
    (128, True, 1, False, 45),
    (128, False, 0, True, 300),
    (64, True, 0, True, 300),
])
def test_options_equal_oracle(qh, oracle, gpu, head_dim, tied, flags, kv_f32, n_prompt):
    qnt = qnt_module()
    hp = _narrow(qnt, n_heads=256 // head_dim, head_dim=head_dim, tied_embeddings=tied, flags=flags)
    tens = qnt.synthetic_q4mix(41 + head_dim + flags, hp)
    orc = oracle_decoder(oracle, hp, tens, ctx_len=512, kv_f32=kv_f32)
    dec = qh.Decoder(hp, tens, ctx_len=512, kv_f32=kv_f32)
    ids = np.random.default_rng(n_prompt).integers(0, hp.vocab_size, n_prompt).astype(np.int32)
    _steps_vs_oracle(oracle, orc, dec, ids, 6, full_every=3)
    pos = n_prompt + 6
    _kv_equal(dec, orc, hp, pos)
    # a second turn: 37 more ids at pos0 > 0, the attention reading cached rows and the chunk's own
    more = np.random.default_rng(n_prompt + 1).integers(0, hp.vocab_size, 37).astype(np.int32)
    r = orc.forward_batch(more, pos, top_k=1)
    dec.prefill(more, pos, top_k=1)
    assert (bits(dec.hidden()) == bits(r["hidden"])).all() and (bits(dec.logits()) == bits(r["logits"])).all()
    _kv_equal(dec, orc, hp, pos + len(more))
    dec.close()


def test_options_one_launch_per_operation_equal_oracle(qh, oracle, gpu, monkeypatch):
    monkeypatch.setenv("QH_DECODER_FUSE", "0")
    qnt = qnt_module()
    hp = _narrow(qnt, tied_embeddings=False, flags=1)
    tens = qnt.synthetic_q4mix(77, hp)
    orc = oracle_decoder(oracle, hp, tens, ctx_len=256, kv_f32=True)
    dec = qh.Decoder(hp, tens, ctx_len=256, kv_f32=True)
    ids = np.random.default_rng(5).integers(0, hp.vocab_size, 40).astype(np.int32)
    _steps_vs_oracle(oracle, orc, dec, ids, 5, full_every=2)
    dec.close()


F32, F16 = 0, 1


@pytest.mark.parametrize("dtype", [F32, F16])
def test_matvec_ref_equals_oracle(qh, oracle, gpu, dtype):
    """qh_matvec_ref: F32 / F16 weights at the decoder's shapes (a last 32-column tile at 1312 columns), ragged row
    ranges, bit for bit against the oracle's matvec_ref."""
    import torch
    for n, k in [(896, 896), (128, 896), (4864, 896), (896, 4864), (70, 1312)]:
        w = (np.random.default_rng(n + k).standard_normal((n, k)) * 0.05).astype(np.float32)
        buf = w.astype(np.float16).view(np.uint8).reshape(-1) if dtype == F16 else w.view(np.uint8).reshape(-1)
        x = (np.random.default_rng(k).standard_normal(k)).astype(np.float32)
        W = qh.DeviceTensor.upload(buf, dtype, n, k)
        xt = torch.from_numpy(x).to(gpu)
        got = qh.matvec_ref(W, xt).cpu().numpy()
        assert (bits(got) == bits(oracle.matvec_f(dtype, n, k, buf, x))).all(), (n, k)
        r0, r1 = 5, n - 3
        part = qh.matvec_ref(W, xt, r0=r0, r1=r1).cpu().numpy()
        assert (bits(part[r0:r1]) == bits(got[r0:r1])).all() and (part[:r0] == 0).all() and (part[r1:] == 0).all()


def _mixed(qnt, synth, hp, seed, emb):
    """q4mix tensors with some matrices unquantized (an F32 k and o projection, an F16 down projection in the last
    layer) and the embedding in `emb`; untied, so the Q8_0 LM head keeps the shortlist."""
    tens = qnt.synthetic_q4mix(seed, hp)
    f32, f16 = qnt.synthetic_dense(seed + 1, hp, F32), qnt.synthetic_dense(seed + 2, hp, F16)
    L = hp.n_layers - 1
    tens["model.layers.0.self_attn.k_proj.weight"] = f32["model.layers.0.self_attn.k_proj.weight"]
    tens["model.layers.0.self_attn.o_proj.weight"] = f32["model.layers.0.self_attn.o_proj.weight"]
    tens[f"model.layers.{L}.mlp.down_proj.weight"] = f16[f"model.layers.{L}.mlp.down_proj.weight"]
    V, D = hp.vocab_size, hp.dim
    if emb == F16:
        tens["model.embed_tokens.weight"] = f16["model.embed_tokens.weight"]
    elif emb == 3:
        tens["model.embed_tokens.weight"] = qnt.TensorRec(3, V, D, synth.q4_tensor(seed + 3, V, D))
    return tens


@pytest.mark.parametrize("kind,fuse", [("f32", "1"), ("f16", "1"), ("mixed_f16_emb", "1"), ("mixed_q4_emb", "1"),
                                       ("mixed_q4_emb", "0")])
def test_unquantized_models_equal_oracle(qh, oracle, synth, gpu, monkeypatch, kind, fuse):
    """Whole models through the decoder against the oracle bit for bit: prompts longer than one chunk, shortlist and
    full-head steps, a second prefill at pos0 > 0."""
    monkeypatch.setenv("QH_DECODER_FUSE", fuse)
    qnt = qnt_module()
    if kind in ("f32", "f16"):
        hp = _narrow(qnt, tied_embeddings=kind == "f32", flags=int(kind == "f16"))
        tens = qnt.synthetic_dense(71, hp, F32 if kind == "f32" else F16)
        kv_f32 = kind == "f16"
    else:
        hp = _narrow(qnt, tied_embeddings=False)
        tens = _mixed(qnt, synth, hp, 73, F16 if kind == "mixed_f16_emb" else 3)
        kv_f32 = False
    orc = oracle_decoder(oracle, hp, tens, ctx_len=256, kv_f32=kv_f32)
    dec = qh.Decoder(hp, tens, ctx_len=256, kv_f32=kv_f32)
    ids = np.random.default_rng(3).integers(0, hp.vocab_size, 45).astype(np.int32)
    _steps_vs_oracle(oracle, orc, dec, ids, 5, full_every=2, shortlist=kind not in ("f32", "f16"))
    pos = 45 + 5
    more = np.random.default_rng(4).integers(0, hp.vocab_size, 33).astype(np.int32)
    r = orc.forward_batch(more, pos, top_k=1)
    dec.prefill(more, pos, top_k=1)
    assert (bits(dec.hidden()) == bits(r["hidden"])).all() and (bits(dec.logits()) == bits(r["logits"])).all()
    dec.close()


@pytest.mark.parametrize("kind", ["options", "dense"])
def test_option_decode_step_graph_replay_equals_eager(qh, oracle, synth, gpu, kind):
    """A decode step of a model on the option paths (untied head, Hadamard down projection, f32 cache; or a model mixing
    F32 / F16 / Q4_0 matrices and a Q4_0 embedding) captured once in a HIP graph and replayed, with eager work between
    the replays: the same tokens as eager steps, and the final hidden state equal to the oracle's."""
    import torch
    qnt = qnt_module()
    if kind == "options":
        hp = _narrow(qnt, tied_embeddings=False, flags=1)
        tens, kv_f32 = qnt.synthetic_q4mix(91, hp), True
    else:
        hp = _narrow(qnt, tied_embeddings=False)
        tens, kv_f32 = _mixed(qnt, synth, hp, 93, 3), False
    dec = qh.Decoder(hp, tens, ctx_len=256, kv_f32=kv_f32)
    ids = np.random.default_rng(6).integers(0, hp.vocab_size, 40).astype(np.int32)
    n = 12
    dec.prefill(ids, 0, top_k=1)
    dec.begin(n + 1)
    for _ in range(n):
        dec.step(top_k=1)
    eager = dec.outputs(n + 1).copy()
    dec.prefill(ids, 0, top_k=1)
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
    orc = oracle_decoder(oracle, hp, tens, ctx_len=256, kv_f32=kv_f32)
    r = orc.forward_batch(ids, 0, top_k=1)
    pos = len(ids)
    for t in eager[:n]:
        r = orc.forward(int(t), pos, top_k=1)
        pos += 1
    assert (bits(dec.hidden()) == bits(r["hidden"])).all()
    dec.close()
