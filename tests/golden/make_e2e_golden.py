#!/usr/bin/env python3
"""Writes the end-to-end golden vectors under tests/golden/ from the reference engine itself.

The synthetic q4mix models are written by quanta.cpp_amd/qnt.py (seeded, the same on every machine) and loaded by the
reference's own Model::load; the token streams come from the reference's `gen --greedy` flow (Session::feed with the
batched 32-token prefill, then Session::generate with the greedy sampler, so the Exact Shortlist Head answers top-1
queries), run through oracle/_ref/libquanta_ref.so (built from the reference sources by oracle/Makefile). Needs that
build, so it runs only where the reference tree is mounted; the .npz files are data.

  e2e_q4mix.npz   the benchmark model (24 layers, vocab 151936, Qwen2.5-0.5B shapes), seed 5: a 512-id prompt
                  uniform over the vocabulary (seed 9), the 256 generated ids, per step the 8-bit head rows the
                  forward read and the exact logit of the chosen id, after the prefill and every step a digest of the
                  final normed hidden state and of its int8 quantization (state_digests, [257][2] uint64), and
                  digests of a few tensors so a GPU host can show it rebuilt the same file. (A random-init model with
                  a tied embedding soon repeats one token; the per-step state digests, head rows and logit bits
                  depend on every operation of every forward.)
  e2e_small.npz   a 2-layer, vocab-4096 model of the same widths (seed 7): 40-id prompt, 24 generated ids, and after
                  the prefill and every decode step the final normed hidden state and its int8 quantization.
  e2e_sampled.npz the benchmark model and prompt in sampling mode, through the reference's Session with the batched
                  prefill: "chat" (head queries and draws from the reference's default SamplerParams -- temperature
                  0.7, top-k 20, top-p 0.8, repetition penalty 1.1 over the whole history -- and seed 0x51A7C0DE)
                  and "gen" (`quanta gen --top-k 20 --repeat-penalty 1.1`: top-k 20 queries with the history as
                  must ids, greedy picks): 256 ids each and the 8-bit head rows of the forward before each pick.

  e2e_options.npz the reference's load-time options on 2-layer, vocab-4096 models of the same widths: an untied LM
                  head, the Hadamard-rotated down projection, the f32 KV cache and all three together; per variant the
                  gen flow's states after every forward (as e2e_small) and one full-head forward's logits digest.

Usage: python tests/golden/make_e2e_golden.py [--small-only | --full-only | --sampled-only | --options-only]
"""
import ctypes as C
import hashlib
import importlib.util
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402


def load_pkg():
    pkg = os.path.join(ROOT, "quanta.cpp_amd")
    spec = importlib.util.spec_from_file_location("quanta_cpp_amd", os.path.join(pkg, "__init__.py"),
                                                  submodule_search_locations=[pkg])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["quanta_cpp_amd"] = mod
    spec.loader.exec_module(mod)
    import quanta_cpp_amd.qnt as qnt
    return qnt


def bind(L):
    L.ref_model_load.restype = C.c_void_p
    L.ref_model_load.argtypes = [C.c_char_p, C.c_int, C.c_int]
    L.ref_model_free.argtypes = [C.c_void_p]
    L.ref_gen.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]
    L.ref_model_forward.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p,
                                    C.c_void_p]
    L.ref_model_forward_batch.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p,
                                          C.c_void_p, C.c_void_p]
    return L


def digest(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).view(np.uint8).tobytes()).hexdigest()


def make_small(qnt, L):
    hp = qnt.HParams(vocab_size=4096, n_layers=2)
    path = "/tmp/quanta_e2e_small.qnt"
    qnt.write_qnt(path, hp, qnt.synthetic_q4mix(7, hp))
    m = L.ref_model_load(path.encode(), 4096, 8)
    assert m, "reference failed to load the small model"
    ids = np.random.default_rng(11).integers(0, hp.vocab_size, 40).astype(np.int32)
    n_gen = 24
    D = hp.dim
    hidden = np.zeros((n_gen + 1, D), np.float32)
    hq = np.zeros((n_gen + 1, D), np.int8)
    hd = np.zeros((n_gen + 1, D // 32), np.float32)
    logits = np.zeros(hp.vocab_size, np.float32)
    out = np.zeros(n_gen, np.int32)
    rows = np.zeros(n_gen + 1, np.int32)
    # the gen flow by hand (Session::feed then greedy Session::generate), recording the state after every forward
    rows[0] = L.ref_model_forward_batch(m, ids.ctypes.data, len(ids), 0, 1, logits.ctypes.data, hidden[0].ctypes.data,
                                        hq[0].ctypes.data, hd[0].ctypes.data)
    pos = len(ids)
    for s in range(n_gen):
        tok = int(np.argmax(logits))  # first maximum over the whole vocabulary (-inf outside the shortlist)
        out[s] = tok
        rows[s + 1] = L.ref_model_forward(m, tok, pos, 1, logits.ctypes.data, hidden[s + 1].ctypes.data,
                                          hq[s + 1].ctypes.data, hd[s + 1].ctypes.data)
        pos += 1
    L.ref_model_free(m)
    # the same stream through the reference's Session, as `quanta gen` runs it
    m = L.ref_model_load(path.encode(), 4096, 8)
    out2 = np.zeros(n_gen, np.int32)
    assert L.ref_gen(m, ids.ctypes.data, len(ids), n_gen, out2.ctypes.data, None, None) == n_gen
    L.ref_model_free(m)
    assert (out == out2).all(), "hand-run gen flow differs from Session::generate"
    np.savez_compressed(os.path.join(HERE, "e2e_small.npz"), seed=np.int32(7), vocab=np.int32(hp.vocab_size),
                        n_layers=np.int32(hp.n_layers), prompt=ids, out=out, head_rows=rows, hidden=hidden, hq=hq, hd=hd)
    os.remove(path)


# The reference's load-time options on a 2-layer, vocabulary-4096 model of the Qwen2.5-0.5B widths (ffn 4864, a
# multiple of 256): an untied LM head (lm_head.weight, model.cpp:16), the Hadamard-rotated down projection
# (FLAG_HADAMARD_DOWN, model.cpp:219, 424; ops_ref.cpp:228-241), the f32 KV cache (--kv-f32, model.cpp:96-104,
# 197-204), and all three together on the q4mix tensors; then unquantized models as the exporter writes them with
# --dtype f32 / f16 (every matrix and the embedding in that dtype: matvec_ref and get_row, ops_ref.cpp:8-27,
# 162-192), tied and untied; (name, seed, tied, flags, kv_f16, dtype: -1 for q4mix, else F32 / F16).
OPTIONS = (("untied", 17, False, 0, True, -1), ("hadamard", 19, True, 1, True, -1), ("kv_f32", 23, True, 0, False, -1),
           ("all", 29, False, 1, False, -1), ("f32", 31, True, 0, True, 0), ("f16", 37, False, 1, True, 1))


def make_options(qnt, L):
    """e2e_options.npz: per variant, the gen flow (batched prefill of a 40-id prompt, 16 greedy shortlist steps) with
    the final normed hidden state, its quantization and the head rows after every forward, then one full-head
    forward's logits (their sha256). An unquantized model quantizes nothing (Model::prepare_input), so its hq / hd
    stay zero."""
    out = {}
    for name, seed, tied, flags, kv_f16, dtype in OPTIONS:
        hp = qnt.HParams(vocab_size=4096, n_layers=2, tied_embeddings=tied, flags=flags)
        path = f"/tmp/quanta_e2e_{name}.qnt"
        qnt.write_qnt(path, hp, qnt.synthetic_q4mix(seed, hp) if dtype < 0 else qnt.synthetic_dense(seed, hp, dtype))
        m = oracle.ref.load_model(path, 4096, 8, kv_f16=kv_f16)
        ids = np.random.default_rng(seed + 1).integers(0, hp.vocab_size, 40).astype(np.int32)
        n_gen = 16
        D = hp.dim
        hidden = np.zeros((n_gen + 1, D), np.float32)
        hq = np.zeros((n_gen + 1, D), np.int8)
        hd = np.zeros((n_gen + 1, D // 32), np.float32)
        logits = np.zeros(hp.vocab_size, np.float32)
        toks = np.zeros(n_gen, np.int32)
        rows = np.zeros(n_gen + 1, np.int32)
        qp = (lambda a: a.ctypes.data) if dtype < 0 else (lambda a: None)  # noqa: E731
        rows[0] = L.ref_model_forward_batch(m, ids.ctypes.data, len(ids), 0, 1, logits.ctypes.data,
                                            hidden[0].ctypes.data, qp(hq[0]), qp(hd[0]))
        pos = len(ids)
        for s in range(n_gen):
            tok = int(np.argmax(logits))
            toks[s] = tok
            rows[s + 1] = L.ref_model_forward(m, tok, pos, 1, logits.ctypes.data, hidden[s + 1].ctypes.data,
                                              qp(hq[s + 1]), qp(hd[s + 1]))
            pos += 1
        tok = int(np.argmax(logits))
        full_rows = L.ref_model_forward(m, tok, pos, 0, logits.ctypes.data, None, None, None)
        assert full_rows == hp.vocab_size
        oracle.ref.free_model(m)
        os.remove(path)
        out.update({f"{name}_seed": np.int32(seed), f"{name}_tied": np.int32(tied), f"{name}_flags": np.int32(flags),
                    f"{name}_dtype": np.int32(dtype),
                    f"{name}_kv_f16": np.int32(kv_f16), f"{name}_prompt": ids, f"{name}_out": toks,
                    f"{name}_head_rows": rows, f"{name}_hidden": hidden, f"{name}_hq": hq, f"{name}_hd": hd,
                    f"{name}_full_token": np.int32(tok), f"{name}_full_logits_sha256": np.array(digest(logits))})
    np.savez_compressed(os.path.join(HERE, "e2e_options.npz"), variants=np.array([o[0] for o in OPTIONS]), **out)


def state_digest(hidden, hq, hd) -> np.ndarray:
    """8 bytes (as uint64) of the sha256 of a forward's final normed hidden state, then of its int8 quantization and
    block scales: a fingerprint of every operation of that forward."""
    h1 = hashlib.sha256(np.ascontiguousarray(hidden, np.float32).tobytes()).digest()[:8]
    h2 = hashlib.sha256(np.ascontiguousarray(hq, np.int8).tobytes() +
                        np.ascontiguousarray(hd, np.float32).tobytes()).digest()[:8]
    return np.frombuffer(h1 + h2, np.uint64)


def make_full(qnt, L):
    hp = qnt.HParams()
    path = "/tmp/quanta_e2e_q4mix.qnt"
    tens = qnt.synthetic_q4mix(5, hp)
    qnt.write_qnt(path, hp, tens)
    m = L.ref_model_load(path.encode(), 4096, 8)
    assert m, "reference failed to load the q4mix model"
    ids = np.random.default_rng(9).integers(0, hp.vocab_size, 512).astype(np.int32)
    out = np.zeros(256, np.int32)
    rows = np.zeros(256, np.int32)
    top = np.zeros(256, np.float32)
    n = L.ref_gen(m, ids.ctypes.data, len(ids), 256, out.ctypes.data, rows.ctypes.data, top.ctypes.data)
    assert n == 256
    L.ref_model_free(m)
    # the same flow by hand (forward_batch, then forward of each greedy token), recording a digest of the final normed
    # hidden state and of its quantization after the prefill and after every decode step: the random-init model soon
    # repeats one token, so the stream alone says little about the forwards behind it
    m = L.ref_model_load(path.encode(), 4096, 8)
    D, V = hp.dim, hp.vocab_size
    logits = np.zeros(V, np.float32)
    hidden = np.zeros(D, np.float32)
    hq = np.zeros(D, np.int8)
    hd = np.zeros(D // 32, np.float32)
    dig = np.zeros((257, 2), np.uint64)
    L.ref_model_forward_batch(m, ids.ctypes.data, len(ids), 0, 1, logits.ctypes.data, hidden.ctypes.data,
                              hq.ctypes.data, hd.ctypes.data)
    dig[0] = state_digest(hidden, hq, hd)
    pos = len(ids)
    for s in range(256):
        tok = int(np.argmax(logits))
        assert tok == out[s], "hand-run gen flow differs from Session::generate"
        L.ref_model_forward(m, tok, pos, 1, logits.ctypes.data, hidden.ctypes.data, hq.ctypes.data, hd.ctypes.data)
        dig[s + 1] = state_digest(hidden, hq, hd)
        pos += 1
    L.ref_model_free(m)
    names = ["model.embed_tokens.weight", "quanta.head_q4", "quanta.head_err", "model.layers.23.mlp.down_proj.weight",
             "model.layers.0.self_attn.q_proj.bias"]
    np.savez_compressed(os.path.join(HERE, "e2e_q4mix.npz"), seed=np.int32(5), prompt=ids, out=out, head_rows=rows,
                        top_logit=top, state_digests=dig,
                        digest_names=np.array(names), digests=np.array([digest(tens[k].data) for k in names]))
    os.remove(path)


SAMPLED_SEED = 0x51A7C0DE


def make_sampled(qnt):
    hp = qnt.HParams()
    path = "/tmp/quanta_e2e_q4mix.qnt"
    tens = qnt.synthetic_q4mix(5, hp)
    qnt.write_qnt(path, hp, tens)
    ids = np.random.default_rng(9).integers(0, hp.vocab_size, 512).astype(np.int32)
    chat = oracle.sampler_params()
    greedy = oracle.sampler_params(temperature=0.0, repeat_penalty=1.0)
    gen_q = oracle.sampler_params(top_k=20, repeat_penalty=1.1)
    res = {}
    for name, (q, sp) in {"chat": (chat, chat), "gen": (gen_q, greedy)}.items():
        m = oracle.ref.load_model(path, 4096, 8)
        out, rows = oracle.ref.gen_sampled(m, ids, 256, q, sp, SAMPLED_SEED)
        oracle.ref.free_model(m)
        assert len(out) == 256
        res[name + "_out"] = out
        res[name + "_rows"] = rows
    np.savez_compressed(os.path.join(HERE, "e2e_sampled.npz"), seed=np.int32(5), prompt=ids,
                        sampler_seed=np.uint64(SAMPLED_SEED), **res)
    os.remove(path)


def main():
    if oracle.ref is None:
        raise SystemExit("oracle/_ref/libquanta_ref.so is missing: run `make -C oracle ref`")
    qnt = load_pkg()
    L = bind(oracle.ref.lib)
    if "--options-only" in sys.argv:
        make_options(qnt, L)
        return
    if "--sampled-only" not in sys.argv:
        if "--full-only" not in sys.argv:
            make_small(qnt, L)
            make_options(qnt, L)
        if "--small-only" not in sys.argv:
            make_full(qnt, L)
    if "--small-only" not in sys.argv and "--full-only" not in sys.argv:
        make_sampled(qnt)
    for f in sorted(os.listdir(HERE)):
        if f.startswith("e2e") and f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
