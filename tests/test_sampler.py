"""The oracle's Sampler::sample restatement against the reference's own Sampler (sampler.cpp:22-85, built from its
sources in oracle/_ref): the chosen id, the penalized logits and the generator state after the draw, bit for bit,
over the parameter space the reference exposes (repetition penalty with a window, temperature, top-k, top-p,
min-p), histories with repeated and out-of-range ids, and shortlist-style logits that are -inf outside a few rows.
Equal logits inside the top-k are avoided: the reference's std::sort leaves their order unspecified (the oracle,
like the GPU sampler, puts the lower id first)."""
import itertools

import numpy as np
import pytest

from oracle import oracle, ref, sampler_params

pytestmark = pytest.mark.skipif(oracle is None, reason="oracle not built")
needs_ref = pytest.mark.skipif(ref is None, reason="the reference build (oracle/_ref) is absent")


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def draw_case(rng, n, n_valid, shortlist):
    logits = (rng.normal(0.0, 2.5, n) * rng.choice([0.3, 1.0, 4.0])).astype(np.float32)
    if shortlist:  # the Exact Shortlist Head's output: exact rows, -inf elsewhere
        keep = rng.choice(n_valid, size=60, replace=False)
        out = np.full(n, -np.inf, np.float32)
        out[keep] = logits[keep]
        logits = out
    hist = rng.integers(-3, n + 5, int(rng.integers(0, 80))).astype(np.int32)
    if hist.size:
        hist[rng.random(hist.size) < 0.3] = hist[0]  # repeats
    return logits, hist


@needs_ref
def test_oracle_sampler_equals_reference_sampler():
    rng = np.random.default_rng(2024)
    grid = itertools.product([0.0, 0.3, 0.7, 1.5], [0, 1, 20, 55], [1.0, 0.8, 0.3], [0.0, 0.05], [1.0, 1.1, 0.8],
                             [0, 7])
    n_cases = 0
    for temp, top_k, top_p, min_p, pen, window in grid:
        shortlist = top_k > 0 and rng.random() < 0.5
        n = 3000
        n_valid = n - int(rng.integers(0, 50))
        logits, hist = draw_case(rng, n, n_valid, shortlist)
        fin = np.sort(logits[:n_valid][np.isfinite(logits[:n_valid])])
        if np.any(np.diff(fin) == 0):
            continue
        if top_k == 0 and not np.all(np.isfinite(logits[:n_valid])):
            continue  # -inf ties would reach the draw's fall-through order
        p = sampler_params(temp, top_k, top_p, min_p, pen, window)
        st = oracle.sampler_seed(int(rng.integers(1, 2**63)))
        for _ in range(3):  # successive draws chain the generator state
            a = oracle.sample(logits, n_valid, hist, p, st)
            b = ref.sample(logits, n_valid, hist, p, st)
            assert a[0] == b[0], (temp, top_k, top_p, min_p, pen, window)
            assert same_bits(a[1], b[1]) and a[2] == b[2]
            st = a[2]
        n_cases += 1
    assert n_cases > 500


@needs_ref
def test_sampler_defaults_many_draws():
    """The reference's defaults (temperature 0.7, top-k 20, top-p 0.8, penalty 1.1), 400 chained draws."""
    rng = np.random.default_rng(7)
    p = sampler_params()
    st = oracle.sampler_seed(0x51A7C0DE)
    hist = list(rng.integers(0, 5000, 30))
    for i in range(400):
        logits = rng.normal(0.0, 3.0, 5000).astype(np.float32)
        a = oracle.sample(logits, 5000, np.array(hist, np.int32), p, st)
        b = ref.sample(logits, 5000, np.array(hist, np.int32), p, st)
        assert a[0] == b[0] and a[2] == b[2], i
        hist.append(a[0])
        st = a[2]


def test_sampler_closed_forms():
    """Cases the mathematics fixes, independent of the reference build."""
    rng = np.random.default_rng(3)
    logits = rng.normal(0.0, 1.0, 500).astype(np.float32)
    # greedy: the first maximum, after the penalty
    g = sampler_params(temperature=0.0, repeat_penalty=1.0)
    assert oracle.sample(logits, 500, [], g, 1)[0] == int(np.argmax(logits))
    top = int(np.argmax(logits))
    pen = sampler_params(temperature=0.0, repeat_penalty=1e9)
    tid, lg, st = oracle.sample(logits, 500, [top], pen, 1)
    assert tid != top and st == 1  # greedy draws nothing
    assert lg[top] == np.float32(logits[top] / np.float32(1e9)) if logits[top] > 0 else True
    # top_k = 1 always returns the maximum, whatever the draw; the generator still advances one step
    one = sampler_params(temperature=0.7, top_k=1, top_p=1.0, repeat_penalty=1.0)
    st = oracle.sampler_seed(99)
    for _ in range(20):
        tid, _, st2 = oracle.sample(logits, 500, [], one, st)
        assert tid == top and st2 != st
        st = st2
    # xorshift64*: the state after one draw from seed 1 (state 1)
    s = 1
    s ^= s >> 12
    s = (s ^ (s << 25)) & (2**64 - 1)
    s ^= s >> 27
    assert oracle.sample(logits, 500, [], one, 1)[2] == s
    # a penalty on an id outside [0, n_valid) changes nothing
    tid, lg, _ = oracle.sample(logits, 400, [450, -1], sampler_params(temperature=0.0, repeat_penalty=2.0), 1)
    assert same_bits(lg, logits)
