"""The Exact Shortlist Head at full strength: 1024 seeded hidden states on the benchmark's 151936 x 896 head, against
the reference's own Model::shortlist_head (engine/src/model.cpp:240-334; tests/golden/head_sweep.npz, written by
tests/golden/make_head_sweep.py from oracle/_ref). Per vector: greedy token and its logit bits, last_head_rows, tau,
no seed tie, and the sets of seed rows and of all rescored rows. On 16 of them, check_head's invariants
(engine/src/checks.cpp:178-239) against the GPU's full 8-bit head: the bound holds on every row, every rescored logit is
bit-identical, the top-1 is the full head's first maximum."""
import hashlib
import os

import numpy as np
import pytest

from conftest import GOLDEN, bits

pytestmark = pytest.mark.gpu


def digest8(a):
    return np.frombuffer(hashlib.sha256(np.ascontiguousarray(a).tobytes()).digest()[:8], np.uint64)[0]


def test_shortlist_head_sweep_1024_vectors(qh, synth, gpu):
    import torch
    g = np.load(os.path.join(GOLDEN, "head_sweep.npz"), allow_pickle=False)
    V, D, N, k = int(g["vocab"]), int(g["dim"]), len(g["top1"]), int(g["top_k"])
    head8, head4, err = synth.shortlist_head(int(g["head_seed"]), V, D)
    h8 = qh.DeviceTensor.upload(head8, qh.Q8_0, V, D)
    h4 = qh.DeviceTensor.upload(head4, qh.Q4_0, V, D)
    he = qh.DeviceTensor.upload(err.view(np.uint8), qh.F16, V, D // 32)
    del head8, head4, err
    x = torch.from_numpy(synth.activations(int(g["x_seed"]), N, D, scale=0.5)).to(gpu)
    xq, xd = qh.quantize_q8(x)
    xqn, xdn = xq.cpu().numpy(), xd.cpu().numpy()
    assert hashlib.sha256(xqn.tobytes() + xdn.tobytes()).hexdigest() == str(g["x_digest"])
    sl = qh.ShortlistHead(h8, h4, he, top_k=k)
    n_seed = k + 8
    for t in range(N):
        sl(xq[t], xd[t])
        st = sl.stats()
        rows = sl.rows[: st["n_rows"]].cpu().numpy()
        assert not st["seed_tie"] and not g["seed_tie"][t], t
        assert st["top1"] == g["top1"][t], (t, st["top1"], g["top1"][t])
        assert np.float32(st["top1_logit"]).tobytes() == g["top1_logit"][t].tobytes(), t
        assert st["n_rows"] == g["n_rows"][t] and st["n_seeds"] == n_seed, t
        assert np.float32(st["tau"]).tobytes() == g["tau"][t].tobytes(), t
        assert digest8(np.sort(rows[:n_seed]).astype(np.int32)) == g["seeds_digest"][t], t
        assert digest8(np.sort(rows).astype(np.int32)) == g["rows_digest"][t], t
        if t % 256 == 0:
            print(f"vector {t}: top1 {st['top1']} rows {st['n_rows']}", flush=True)
    for t in range(16):
        full = qh.matvec_q(h8, xq[t], xd[t])
        sl(xq[t], xd[t])
        st = sl.stats()
        coarse, upper, lg, fl = (a.cpu().numpy() for a in (sl.coarse, sl.upper, sl.logits, full))
        assert (np.abs(fl - coarse) <= upper - coarse).all(), t  # the bound, as check_head evaluates it
        exact = lg != -np.inf
        assert (bits(lg[exact]) == bits(fl[exact])).all(), t
        assert st["top1"] == int(np.argmax(fl)), t
