"""Pins the oracle's decoder restatement (oracle/quanta_oracle.c, qo_decoder_*) bit for bit: against the golden
states the reference engine wrote for a small synthetic model (tests/golden/e2e_small.npz) and for its load-time
options (an untied LM head, the Hadamard-rotated down projection, the f32 KV cache: tests/golden/e2e_options.npz),
against the reference build itself where it is present (oracle/_ref), and its float->half rounding against numpy's.
No GPU."""
import ctypes as C
import os

import numpy as np
import pytest

from conftest import GOLDEN, bits
from decoder_util import logits_sha256, option_model, oracle_decoder, qnt_module


def test_f32_to_f16_rounding(oracle):
    rng = np.random.default_rng(3)
    u = np.concatenate([rng.integers(0, 1 << 32, 200000, dtype=np.uint64).astype(np.uint32),
                        np.arange(0x33000000, 0x33000000 + 4096, dtype=np.uint32),   # around 2^-25
                        np.arange(0x387fe000, 0x38802000, dtype=np.uint32),          # the normal/subnormal edge
                        np.arange(0x477fe000, 0x47801000, dtype=np.uint32)])         # around 65504 and 65520
    f = u.view(np.float32)
    fin = np.isfinite(f)
    with np.errstate(over="ignore"):
        want = f[fin].astype(np.float16).view(np.uint16)
    got = np.array([oracle.f32_to_f16(float(x)) for x in f[fin]], np.uint16)
    assert (got == want).all(), np.nonzero(got != want)[0][:8]


@pytest.fixture(scope="module")
def small():
    qnt = qnt_module()
    g = np.load(os.path.join(GOLDEN, "e2e_small.npz"), allow_pickle=False)
    hp = qnt.HParams(vocab_size=int(g["vocab"]), n_layers=int(g["n_layers"]))
    return qnt, hp, qnt.synthetic_q4mix(int(g["seed"]), hp), g


def test_oracle_decoder_matches_golden_states(oracle, small):
    qnt, hp, tens, g = small
    dec = oracle_decoder(oracle, hp, tens)
    r = dec.forward_batch(g["prompt"], 0)
    pos = len(g["prompt"])
    for s in range(len(g["out"]) + 1):
        assert r["rows"] == int(g["head_rows"][s]), s
        assert (bits(r["hidden"]) == bits(g["hidden"][s])).all(), f"hidden state after step {s}"
        assert (r["hq"] == g["hq"][s]).all() and (bits(r["hd"]) == bits(g["hd"][s])).all()
        if s == len(g["out"]):
            break
        tok = int(np.argmax(r["logits"]))
        assert tok == int(g["out"][s]), s
        r = dec.forward(tok, pos)
        pos += 1


@pytest.fixture(scope="module")
def ref():
    import oracle as o
    if o.ref is None:
        pytest.skip("oracle/_ref is not built (the reference sources are not mounted here)")
    L = o.ref.lib
    L.ref_model_load.restype = C.c_void_p
    L.ref_model_load.argtypes = [C.c_char_p, C.c_int, C.c_int]
    L.ref_model_free.argtypes = [C.c_void_p]
    L.ref_model_forward.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p,
                                    C.c_void_p]
    L.ref_model_forward_batch.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p,
                                          C.c_void_p, C.c_void_p]
    return L


def test_oracle_decoder_equals_reference_build(oracle, ref, tmp_path):
    """Another seed, full-head and shortlist steps, a prompt longer than one 32-token chunk, logits compared."""
    qnt = qnt_module()
    hp = qnt.HParams(vocab_size=3072, n_layers=3)
    tens = qnt.synthetic_q4mix(23, hp)
    path = str(tmp_path / "m.qnt")
    qnt.write_qnt(path, hp, tens)
    m = ref.ref_model_load(path.encode(), 512, 4)
    assert m
    dec = oracle_decoder(oracle, hp, tens, ctx_len=512)
    V, D = hp.vocab_size, hp.dim
    ids = np.random.default_rng(5).integers(0, V, 45).astype(np.int32)
    lg, h = np.empty(V, np.float32), np.empty(D, np.float32)
    rows = ref.ref_model_forward_batch(m, ids.ctypes.data, len(ids), 0, 1, lg.ctypes.data, h.ctypes.data, None, None)
    r = dec.forward_batch(ids, 0, top_k=1)
    assert r["rows"] == rows and (bits(r["hidden"]) == bits(h)).all() and (bits(r["logits"]) == bits(lg)).all()
    pos = len(ids)
    for step in range(6):
        top_k = 0 if step % 3 == 2 else 1
        tok = int(np.argmax(lg))
        rows = ref.ref_model_forward(m, tok, pos, top_k, lg.ctypes.data, h.ctypes.data, None, None)
        r = dec.forward(tok, pos, top_k=top_k)
        assert r["rows"] == rows, step
        assert (bits(r["hidden"]) == bits(h)).all(), step
        assert (bits(r["logits"]) == bits(lg)).all(), step
        pos += 1
    ref.ref_model_free(m)


def test_oracle_second_turn_prefill_equals_reference_build(oracle, ref, tmp_path):
    """check_batch's second turn (engine/src/checks.cpp:148-176; session.cpp:13-31): a prefill at pos0 > 0 over a cache
    filled by an earlier prefill, directly (pos0 = 40, n = 45) and after three decode steps (pos0 = 43, not a multiple
    of the V cache's 8-position blocks); hidden state, logits and head rows equal the reference build's."""
    qnt = qnt_module()
    hp = qnt.HParams(vocab_size=3072, n_layers=3)
    tens = qnt.synthetic_q4mix(23, hp)
    path = str(tmp_path / "m.qnt")
    qnt.write_qnt(path, hp, tens)
    V, D = hp.vocab_size, hp.dim
    ids = np.random.default_rng(31).integers(0, V, 85).astype(np.int32)
    lg, h = np.empty(V, np.float32), np.empty(D, np.float32)
    for n_steps in (0, 3):
        m = ref.ref_model_load(path.encode(), 512, 4)
        dec = oracle_decoder(oracle, hp, tens, ctx_len=512)
        ref.ref_model_forward_batch(m, ids.ctypes.data, 40, 0, 1, lg.ctypes.data, h.ctypes.data, None, None)
        r = dec.forward_batch(ids[:40], 0, top_k=1)
        assert (bits(r["logits"]) == bits(lg)).all()
        pos = 40
        for _ in range(n_steps):
            tok = int(np.argmax(lg))
            ref.ref_model_forward(m, tok, pos, 1, lg.ctypes.data, h.ctypes.data, None, None)
            r = dec.forward(tok, pos, top_k=1)
            assert (bits(r["logits"]) == bits(lg)).all()
            pos += 1
        second = np.ascontiguousarray(ids[40:85])
        rows = ref.ref_model_forward_batch(m, second.ctypes.data, 45, pos, 1, lg.ctypes.data, h.ctypes.data, None,
                                           None)
        r = dec.forward_batch(second, pos, top_k=1)
        assert r["rows"] == rows and (bits(r["hidden"]) == bits(h)).all() and (bits(r["logits"]) == bits(lg)).all()
        ref.ref_model_free(m)


@pytest.mark.parametrize("name", ["untied", "hadamard", "kv_f32", "all", "f32", "f16"])
def test_oracle_decoder_options_match_golden(oracle, name):
    """The gen flow of each load-time option and of the unquantized models: every forward's final normed state,
    quantization (quantized models only: an unquantized one has none), head rows and token as the reference wrote
    them, then one full-head forward's logits."""
    g = np.load(os.path.join(GOLDEN, "e2e_options.npz"), allow_pickle=False)
    hp, tens, kv_f32 = option_model(g, name)
    dec = oracle_decoder(oracle, hp, tens, ctx_len=4096, kv_f32=kv_f32)
    prompt = g[f"{name}_prompt"]
    r = dec.forward_batch(prompt, 0, top_k=1)
    pos = len(prompt)
    for s in range(len(g[f"{name}_out"]) + 1):
        assert (bits(r["hidden"]) == bits(g[f"{name}_hidden"][s])).all(), (name, s)
        if int(g[f"{name}_dtype"]) < 0:
            assert (r["hq"] == g[f"{name}_hq"][s]).all() and (bits(r["hd"]) == bits(g[f"{name}_hd"][s])).all(), (name, s)
        assert r["rows"] == int(g[f"{name}_head_rows"][s]), (name, s)
        tok = oracle.argmax(r["logits"])
        if s < len(g[f"{name}_out"]):
            assert tok == int(g[f"{name}_out"][s]), (name, s)
            r = dec.forward(tok, pos, top_k=1)
            pos += 1
    assert tok == int(g[f"{name}_full_token"])
    r = dec.forward(tok, pos, top_k=0)
    assert logits_sha256(r["logits"]) == str(g[f"{name}_full_logits_sha256"])
