"""GPU parity of the prefill stack (qh_decoder_set_prefill_stack): prompts taken through each layer's norms and
matmuls `stack` tokens at a time (the matmul tile kernels at M up to the stack), attention in 32-token sub-chunks
in order. Every hidden state, logit, row count and KV cache row must equal the oracle's (which runs the reference's
32-token chunks, model.cpp:349-361) bit for bit, for full and partial stacks, second turns at pos0 > 0, the
load-time options and the benchmark model's 256-token stream.
"""
import os

import numpy as np
import pytest

from conftest import GOLDEN, bits
from decoder_util import oracle_decoder, qnt_module
from test_gpu_decoder import _steps_vs_oracle, state_digest
from test_gpu_options import _kv_equal, _narrow

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("stack", [64, 96, 512])
def test_prefill_stack_equals_oracle(qh, oracle, gpu, stack):
    """Prompts of 77 and 300 tokens (one partial stack, or several, the last partial), decode steps after them, and a
    second turn of 45 tokens at pos0 > 0: states, logits, rows and every cache row equal the oracle's."""
    qnt = qnt_module()
    hp = qnt.HParams(vocab_size=3072, n_layers=3)
    tens = qnt.synthetic_q4mix(23, hp)
    for n_prompt in (77, 300):
        orc = oracle_decoder(oracle, hp, tens, ctx_len=512)
        dec = qh.Decoder(hp, tens, ctx_len=512)
        dec.set_prefill_stack(stack)
        ids = np.random.default_rng(n_prompt).integers(0, hp.vocab_size, n_prompt).astype(np.int32)
        print(f"stack {stack}, prompt {n_prompt}", flush=True)
        _steps_vs_oracle(oracle, orc, dec, ids, 4, full_every=2)
        pos = n_prompt + 4
        _kv_equal(dec, orc, hp, pos)
        more = np.random.default_rng(n_prompt + 1).integers(0, hp.vocab_size, 45).astype(np.int32)
        r = orc.forward_batch(more, pos, top_k=1)
        dec.prefill(more, pos, top_k=1)
        assert (bits(dec.hidden()) == bits(r["hidden"])).all() and (bits(dec.logits()) == bits(r["logits"])).all()
        assert dec.stats()["n_rows"] == r["rows"]
        _kv_equal(dec, orc, hp, pos + len(more))
        dec.close()


@pytest.mark.parametrize("head_dim,tied,flags,kv_f32", [(64, False, 1, True), (128, True, 1, False)])
def test_prefill_stack_options_equal_oracle(qh, oracle, gpu, head_dim, tied, flags, kv_f32):
    """The load-time options under a 128-token stack: an untied LM head, the Hadamard-rotated down projection (its
    SwiGLU kernel over the stack), the f32 cache and head_dim 128."""
    qnt = qnt_module()
    hp = _narrow(qnt, n_heads=256 // head_dim, head_dim=head_dim, tied_embeddings=tied, flags=flags)
    tens = qnt.synthetic_q4mix(41 + head_dim + flags, hp)
    orc = oracle_decoder(oracle, hp, tens, ctx_len=512, kv_f32=kv_f32)
    dec = qh.Decoder(hp, tens, ctx_len=512, kv_f32=kv_f32)
    dec.set_prefill_stack(128)
    ids = np.random.default_rng(300).integers(0, hp.vocab_size, 300).astype(np.int32)
    _steps_vs_oracle(oracle, orc, dec, ids, 3, full_every=3)
    _kv_equal(dec, orc, hp, 303)
    dec.close()


def test_prefill_stack_change_keeps_state(qh, oracle, gpu):
    """Switching the stack between prefills (the work buffers move) leaves the cache and the next prefill exact, and
    switching back to 32 restores the reference's chunks."""
    qnt = qnt_module()
    hp = qnt.HParams(vocab_size=3072, n_layers=2)
    tens = qnt.synthetic_q4mix(29, hp)
    orc = oracle_decoder(oracle, hp, tens, ctx_len=512)
    dec = qh.Decoder(hp, tens, ctx_len=512)
    ids = np.random.default_rng(3).integers(0, hp.vocab_size, 200).astype(np.int32)
    pos = 0
    for stack, n in ((256, 70), (32, 50), (1024, 80)):
        dec.set_prefill_stack(stack)
        r = orc.forward_batch(ids[pos:pos + n], pos, top_k=1)
        dec.prefill(ids[pos:pos + n], pos, top_k=1)
        assert (bits(dec.hidden()) == bits(r["hidden"])).all() and (bits(dec.logits()) == bits(r["logits"])).all()
        hq, hd = dec.hq()
        assert hq.shape == (hp.dim,) and np.isfinite(hd).all()
        pos += n
    _kv_equal(dec, orc, hp, pos)
    dec.close()


def test_prefill_stack_q4mix_stream_equals_reference(qh, gpu):
    """The benchmark model with the whole 512-token prompt as one stack: the 256 greedy tokens, each forward's chosen
    logit and final-state digest equal the reference's gen stream (tests/golden/e2e_q4mix.npz)."""
    qnt = qnt_module()
    g = np.load(os.path.join(GOLDEN, "e2e_q4mix.npz"), allow_pickle=False)
    hp = qnt.HParams()
    tens = qnt.synthetic_q4mix(int(g["seed"]), hp)
    dec = qh.Decoder(hp, tens, ctx_len=4096)
    del tens
    dec.set_prefill_stack(512)
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
    assert (dec.outputs(n_gen) == g["out"]).all()
    assert (np.array(digs) == g["state_digests"]).all()
    assert rows == g["head_rows"].tolist()
    assert (bits(np.array(tops, np.float32)) == bits(g["top_logit"])).all()


def test_prefill_stack_fused_swiglu_q8_mlp_equals_oracle(qh, oracle, gpu):
    """The stack's gate / up launch with the SwiGLU epilogue over Q8_0 MLP weights (the q4mix model with its gate, up
    and down matrices re-drawn as Q8_0), stacks of 128 and 256 over a 300-token prompt (full and partial 32-token
    tiles): states, logits, rows and every cache row equal the oracle's."""
    from quanta_cpp_amd import synth
    qnt = qnt_module()
    hp = qnt.HParams(vocab_size=3072, n_layers=2)
    tens = qnt.synthetic_q4mix(31, hp)
    D, F = hp.dim, hp.ffn_dim
    for l in range(hp.n_layers):
        p = f"model.layers.{l}."
        tens[p + "mlp.gate_proj.weight"] = qnt.TensorRec(2, F, D, synth.q8_tensor(700 + l, F, D))
        tens[p + "mlp.up_proj.weight"] = qnt.TensorRec(2, F, D, synth.q8_tensor(710 + l, F, D))
        tens[p + "mlp.down_proj.weight"] = qnt.TensorRec(2, D, F, synth.q8_tensor(720 + l, D, F))
    ids = np.random.default_rng(8).integers(0, hp.vocab_size, 300).astype(np.int32)
    for stack in (128, 256):
        orc = oracle_decoder(oracle, hp, tens, ctx_len=512)
        dec = qh.Decoder(hp, tens, ctx_len=512)
        dec.set_prefill_stack(stack)
        _steps_vs_oracle(oracle, orc, dec, ids, 3, full_every=3)
        _kv_equal(dec, orc, hp, 303)
        dec.close()
