"""The sampling-mode session (Session::feed + Session::generate with head queries built by Session::head_query and
tokens drawn by Sampler::sample, session.cpp:13-79, sampler.cpp:10-85) restated over the oracle's decoder and
sampler, pinned against the reference's own Session run from its sources (oracle/_ref) on a small synthetic model:
the chat flow (queries and draws from the same parameters) and `quanta gen` with sampling options (top-k 20 queries
with the history as must ids, greedy picks). No GPU."""
import os

import numpy as np
import pytest

from decoder_util import oracle_decoder, oracle_session, qnt_module
from oracle import ref, sampler_params

needs_ref = pytest.mark.skipif(ref is None, reason="the reference build (oracle/_ref) is absent")

FLOWS = {
    "chat_defaults": (sampler_params(), sampler_params(), 0x51A7C0DE),
    "chat_window_minp": (sampler_params(0.9, 40, 0.95, 0.02, 1.3, 12), sampler_params(0.9, 40, 0.95, 0.02, 1.3, 12),
                         77),
    "gen_topk20_greedy": (sampler_params(top_k=20, repeat_penalty=1.1), None, 1),
    "greedy_penalty": (sampler_params(temperature=0.0, repeat_penalty=1.5), sampler_params(temperature=0.0,
                                                                                          repeat_penalty=1.5), 3),
}


@pytest.fixture(scope="module")
def small_model(tmp_path_factory):
    qnt = qnt_module()
    hp = qnt.HParams(vocab_size=3000, n_layers=2)
    tens = qnt.synthetic_q4mix(13, hp)
    path = str(tmp_path_factory.mktemp("qnt") / "small.qnt")
    qnt.write_qnt(path, hp, tens)
    return qnt, hp, tens, path


@needs_ref
@pytest.mark.parametrize("flow", sorted(FLOWS))
def test_oracle_session_equals_reference_session(oracle, small_model, flow):
    qnt, hp, tens, path = small_model
    query, sampler, seed = FLOWS[flow]
    prompt = np.random.default_rng(17).integers(0, hp.vocab_size, 45).astype(np.int32)
    prompt[5:25] = prompt[:20]  # repeats for the penalty
    n_gen = 30
    m = ref.load_model(path, 256, 4)
    try:
        greedy = sampler_params(temperature=0.0, repeat_penalty=1.0)
        want, _ = ref.gen_sampled(m, prompt, n_gen, query, sampler if sampler is not None else greedy, seed)
    finally:
        ref.free_model(m)
    dec = oracle_decoder(oracle, hp, tens, ctx_len=256)
    got, _ = oracle_session(oracle, dec, prompt, n_gen, query, sampler, seed, hp.vocab_size)
    assert got == want.tolist()
