"""Helpers shared by the decoder tests: the synthetic-model module and the oracle decoder over a tensor set."""
from conftest import load_package


def qnt_module():
    load_package()
    import quanta_cpp_amd.qnt as qnt
    return qnt


def oracle_decoder(oracle, hp, tensors, ctx_len=None, kv_f32=False):
    return oracle.decoder_for(hp, tensors, ctx_len, kv_f32=kv_f32)


def option_model(g, name):
    """The model of one variant of tests/golden/e2e_options.npz: (HParams, tensors, kv_f32)."""
    qnt = qnt_module()
    hp = qnt.HParams(vocab_size=4096, n_layers=2, tied_embeddings=bool(g[f"{name}_tied"]),
                     flags=int(g[f"{name}_flags"]))
    seed, dtype = int(g[f"{name}_seed"]), int(g[f"{name}_dtype"])
    tens = qnt.synthetic_q4mix(seed, hp) if dtype < 0 else qnt.synthetic_dense(seed, hp, dtype)
    return hp, tens, not bool(g[f"{name}_kv_f16"])


def logits_sha256(logits):
    import hashlib
    import numpy as np
    return hashlib.sha256(np.ascontiguousarray(logits, np.float32).view(np.uint8).tobytes()).hexdigest()


def must_window(hist, params):
    """Session::head_query's must ids (session.cpp:63-79): the history window when the penalty is on, else None."""
    if params is None or params.repeat_penalty == 1.0:
        return None
    w = params.repeat_window
    return list(hist[-w:]) if (w > 0 and len(hist) > w) else list(hist)


def query_top_k(params, default=1):
    """Session::head_query's top_k: 1 when greedy, else the sampler's top_k (0 means the full head)."""
    if params is None:
        return default
    return 1 if params.temperature <= 0 else params.top_k


def oracle_session(oracle, dec, prompt, n_gen, query, sampler, seed, vocab):
    """The oracle's restatement of a batched-prefill Session (session.cpp:13-52): Session::feed, then
    Session::generate with Sampler(sampler, seed) (None: greedy argmax), head queries built from `query`.
    Returns the n_gen chosen ids; out[0] comes from the prompt's logits, out[i] from the forward of out[i-1]."""
    import numpy as np
    hist = [int(t) for t in prompt]
    k = query_top_k(query)
    dec.set_must(must_window(hist, query))
    r = dec.forward_batch(np.asarray(prompt, np.int32), 0, top_k=k)
    state = oracle.sampler_seed(seed)
    out = []
    pos = len(prompt)
    for i in range(n_gen):
        if sampler is None:
            tid = oracle.argmax(r["logits"], vocab)
        else:
            tid, _, state = oracle.sample(r["logits"], vocab, np.asarray(hist, np.int32), sampler, state)
        out.append(tid)
        hist.append(tid)
        if i + 1 == n_gen:
            break
        dec.set_must(must_window(hist, query))
        r = dec.forward(tid, pos, top_k=k)
        pos += 1
    dec.set_must(None)
    return out, state
