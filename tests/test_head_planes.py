"""CPU pins of the oracle's nibble-plane shortlist head (qo_head_planes, qo_shortlist_planes).

The variant is the scope's "nibble-plane shortlist": the Q8_0 head's int8 values stored as a high and a low nibble
plane, the screen reading the high plane only, with the analytic bound 8 * d_b * |x_b|_1 (reference
research/head_deep.py:68-78 "hi4, analytic bound", docs/PROGRESS.md:121-130), run through Model::shortlist_head's
procedure (engine/src/model.cpp:240-334). The reference has no engine code for it (only the research script, which
needs a checkpoint), so the oracle is pinned here by what the mathematics fixes:

- the layout decodes back to the Q8_0 values, q = 16 h + l, h = floor(q / 16), for every int8 value;
- the screen's coarse scores and bounds equal an independent numpy evaluation of their closed forms, bit for bit;
- the bound holds for every row against the exact Q8_0 logits of the oracle's matvec_q (itself pinned to the
  reference build), adversarial rows (every low nibble 0 or 15, the extreme codes) included;
- the rows it returns are the seeds, candidates and must ids the procedure defines, recomputed in numpy from its
  outputs, every rescored logit is the full Q8_0 head's logit and the top-1 is the full head's first argmax.
"""
import numpy as np
import pytest

from conftest import bits


def _fma32(a, b, c):
    """fmaf on float32 arrays through float64: the product of two float32 values is exact in float64, so only the
    sum rounds before the final rounding to float32 (a double rounding that can only matter on an exact float32
    midpoint after a rounded float64 sum)."""
    return (a.astype(np.float64) * b.astype(np.float64) + c.astype(np.float64)).astype(np.float32)


def _adversarial_head(synth, V, D, seed):
    """A Q8_0 head whose first rows have every low nibble 0 (q = 16 h), then every low nibble 15, then only the
    extreme codes -128 / 127 (|q - (16 h + 8)| at its maximum 8), the rest uniform."""
    head8 = synth.q8_tensor(seed, V, D).copy()
    q = head8[: V * D].view(np.int8).reshape(V, D)
    rng = np.random.default_rng(seed)
    h = rng.integers(-8, 8, (8, D))
    q[0:8] = 16 * h
    q[8:16] = 16 * h + 15
    q[16:24] = np.where(rng.random((8, D)) < 0.5, -128, 127)
    return head8


def test_planes_layout_every_value(oracle):
    V, D = 64, 128
    q = np.tile(np.arange(-128, 128, dtype=np.int8), V * D // 256)
    np.random.default_rng(1).shuffle(q)
    scales = np.random.default_rng(2).integers(0, 0x7c00, V * D // 32).astype(np.uint16)
    head8 = np.concatenate([q.view(np.uint8), scales.view(np.uint8)])
    planes = oracle.head_planes(head8, V, D)
    assert planes.size == head8.size
    n = V * D
    hi = planes[: n // 2].reshape(-1, 16)
    lo = planes[n // 2: n].reshape(-1, 16)
    h = np.concatenate([(hi & 15).astype(np.int32), (hi >> 4).astype(np.int32)], axis=1) - 8  # elements 0-15, 16-31
    l = np.concatenate([(lo & 15).astype(np.int32), (lo >> 4).astype(np.int32)], axis=1)
    qq = q.reshape(-1, 32).astype(np.int32)
    assert (16 * h + l == qq).all()
    assert (h == np.floor_divide(qq, 16)).all() and (h >= -8).all() and (h <= 7).all()
    assert (l >= 0).all() and (l <= 15).all()
    assert np.array_equal(planes[n:], head8[n:])  # scales unchanged


def _screen_closed_form(head8, V, D, xq, xd):
    """coarse and upper of the nibble-plane screen from their definitions, in numpy."""
    nb = D // 32
    q = head8[: V * D].view(np.int8).reshape(V, nb, 32).astype(np.int64)
    d = head8[V * D:].view(np.float16).astype(np.float32).reshape(V, nb)
    x = xq.reshape(nb, 32).astype(np.int64)
    mid = 16 * np.floor_divide(q, 16) + 8
    s = np.einsum("vbi,bi->vb", mid, x)
    coarse = np.zeros(V, np.float32)
    bound = np.zeros(V, np.float32)
    l1 = np.abs(x).sum(1).astype(np.float32)
    bop = (np.float32(8.0) * xd.astype(np.float32)) * l1
    for b in range(nb):
        p = s[:, b].astype(np.float32) * d[:, b]
        coarse = _fma32(p, np.full(V, xd[b], np.float32), coarse)
        bound = _fma32(d[:, b], np.full(V, bop[b], np.float32), bound)
    bound = _fma32(bound, np.full(V, np.float32(1.001), np.float32), np.full(V, np.float32(1e-5), np.float32))
    return coarse, coarse + bound


@pytest.mark.parametrize("seed", [3, 4])
def test_planes_screen_closed_form_and_bound(oracle, synth, seed):
    V, D = 3001, 896
    head8 = _adversarial_head(synth, V, D, 20 + seed)
    planes = oracle.head_planes(head8, V, D)
    x = synth.activations(30 + seed, 2, D, scale=0.5)
    x[1] = np.abs(x[1])  # one-signed: the rows with every low nibble 0 miss by exactly the bound
    for t in range(2):
        xq, xd = oracle.quantize_q8(x[t:t + 1])
        o = oracle.shortlist_planes(planes, V, D, xq[0], xd[0], top_k=1)
        coarse, upper = _screen_closed_form(head8, V, D, xq[0], xd[0])
        assert (bits(o["coarse"]) == bits(coarse)).all()
        assert (bits(o["upper"]) == bits(upper)).all()
        exact = oracle.matvec_q(2, V, D, head8, xq[0], xd[0])
        assert (o["upper"] >= exact).all(), "bound violated"
        if t == 1:  # the bound is attained: q - (16 h + 8) = -8 everywhere on rows 0-7, all x_i >= 0
            slack = (o["upper"] - o["coarse"])[:8]
            assert (np.abs(exact - o["coarse"])[:8] > 0.99 * slack).all()


@pytest.mark.parametrize("top_k,n_valid,must", [(1, 0, None), (20, 0, None), (5, 2500, [7, 7, 2999, 100, -1, 2600]),
                                                (64, 0, list(range(0, 3001, 97)))])
def test_planes_procedure(oracle, synth, top_k, n_valid, must):
    V, D = 3001, 896
    head8 = synth.q8_tensor(24, V, D)
    planes = oracle.head_planes(head8, V, D)
    x = synth.activations(35, 1, D, scale=0.5)
    xq, xd = oracle.quantize_q8(x)
    o = oracle.shortlist_planes(planes, V, D, xq[0], xd[0], top_k=top_k, n_valid=n_valid, must=must)
    exact = oracle.matvec_q(2, V, D, head8, xq[0], xd[0])
    nv = n_valid if 0 < n_valid < V else V
    must = must or []
    is_must = np.zeros(V, bool)
    for m in must:
        if 0 <= m < nv:
            is_must[m] = True
    elig = np.flatnonzero(~is_must[:nv])
    order = elig[np.lexsort((elig, -o["coarse"][elig]))]  # best coarse first, lower row on ties
    seeds = order[: top_k + 8]
    tau = np.sort(exact[seeds])[::-1][top_k - 1]
    assert np.float32(o["tau"]).tobytes() == np.float32(tau).tobytes()
    cand = [r for r in range(nv) if not is_must[r] and r not in set(seeds.tolist()) and o["upper"][r] >= tau]
    firsts = []
    for m in must:
        if 0 <= m < nv and m not in firsts:
            firsts.append(m)
    assert o["rows"].tolist() == seeds.tolist() + cand + firsts
    rows = o["rows"]
    assert (bits(o["logits"][rows]) == bits(exact[rows])).all()
    rest = np.setdiff1d(np.arange(V), rows)
    assert np.isneginf(o["logits"][rest]).all()
    best = oracle.argmax(exact, nv) if not must else None
    if best is not None:
        assert oracle.argmax(o["logits"], nv) == best
