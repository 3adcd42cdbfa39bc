"""GPU parity of the decoder's load-time options (Model::load, reference model.cpp:10-106), through the C-ABI:

* an untied LM head (lm_head.weight, model.cpp:16), the Hadamard-rotated down projection (FLAG_HADAMARD_DOWN,
  model.cpp:219, 424), the f32 KV cache (--kv-f32, model.cpp:96-104) and all three together, each on a 2-layer,
  vocabulary-4096 model: after the batched prefill and every greedy decode step, the final normed hidden state, its
  quantization, the head rows and the token equal what the reference engine wrote (tests/golden/e2e_options.npz),
  bit for bit; then one full-head step's logits equal the reference's (sha256) and its greedy token;
* narrower models with head_dim 64 and 128 against the oracle's decoder bit for bit, with prompts longer than one
  32-token chunk, a second prefill at pos0 > 0 (cached rows and chunk rows in one attention), contexts past one LDS
  stage of V rows, shortlist and full-head steps, and the f32 cache itself compared row for row;
* the same with one launch per operation (QH_DECODER_FUSE=0).
"""
import os

import numpy as np
import pytest

from conftest import GOLDEN, bits
from decoder_util import logits_sha256, option_model, oracle_decoder, qnt_module
from test_gpu_decoder import _steps_vs_oracle

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["untied", "hadamard", "kv_f32", "all"])
def test_options_match_reference_states(qh, gpu, name):
    g = np.load(os.path.join(GOLDEN, "e2e_options.npz"), allow_pickle=False)
    hp, tens, kv_f32 = option_model(g, name)
    dec = qh.Decoder(hp, tens, ctx_len=256, kv_f32=kv_f32)
    dec.prefill(g[f"{name}_prompt"], 0, top_k=1)
    n_gen = len(g[f"{name}_out"])
    dec.begin(n_gen + 2)
    for s in range(n_gen + 1):
        assert dec.stats()["n_rows"] == int(g[f"{name}_head_rows"][s]), (name, s)
        assert (bits(dec.hidden()) == bits(g[f"{name}_hidden"][s])).all(), f"{name}: hidden state after step {s}"
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
