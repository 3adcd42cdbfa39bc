#!/usr/bin/env python3
"""Benchmark of the quantized matmul hot path on one MI355X.

Headline (one JSON line on stdout): end-to-end greedy decode of a random-init q4mix model with Qwen2.5-0.5B shapes
(configuration 5): a 512-token prompt in 32-token prefill chunks, then 256 greedy decode steps, every kernel of
the path hand-written HIP (Q8_0 attention / Q4_0 MLP GEMVs with their norms fused, attention, Exact Shortlist
Head). A "step" is one decode step (one token): one replay of a HIP graph holding the captured step. `value` is
decode tokens/s between two HIP events on the replay stream; the generated stream is checked against the reference
engine's own (tests/golden/e2e_q4mix.npz). Prefill tok/s is in `config`.

`roofline` covers the decode step's weight GEMV at its real shapes: Q4_0 gate/up 4864x896 + down 896x4864, batch 1,
over a rotation of distinct weight copies (>= 1 GiB, four times the 256 MB Infinity Cache) so every byte comes
from HBM; algorithmic bytes per launch (0.5625*N*K weights+scales + 1.125*K activation + 4*N output) / average
launch duration, from HIP events around the graph-replayed rotation. `traffic` is the measured HBM bytes per launch
when profiles/q4_gemv_traffic.txt holds rocprofv3 counter readings, else null.
`cpu_baseline` runs the reference engine itself (built from its sources, oracle/_ref) on the host cores over a
bounded sample of the same workload, or the oracle's C restatement where that build is absent.
`extra` adds the other configurations: Q8_0 / Q4_0 GEMV shapes cold and hot, prefill matmuls at M = 32/128/512,
the Exact Shortlist Head against the full 8-bit head, and the reference CPU GEMV.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-extra] [--no-cpu] [--e2e-only]
"""
import argparse
import importlib.util
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
METRIC = "decode tok/s q4mix Qwen2.5-0.5B-shape; Q8/Q4 GEMV GB/s vs HBM peak"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
GIB = 1 << 30


def load_package():
    if "quanta_cpp_amd" in sys.modules:
        return sys.modules["quanta_cpp_amd"]
    pkg_dir = os.path.join(ROOT, "quanta.cpp_amd")
    spec = importlib.util.spec_from_file_location("quanta_cpp_amd", os.path.join(pkg_dir, "__init__.py"),
                                                  submodule_search_locations=[pkg_dir])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["quanta_cpp_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def gemv_bytes(dtype, n, k):
    w = 1.0625 if dtype == 2 else 0.5625
    return w * n * k + 1.125 * k + 4.0 * n


class Rotation:
    """R device copies of one synthetic .qnt tensor, laid out back to back (256-byte aligned)."""

    def __init__(self, qh, torch, host, dtype, rows, cols, copies):
        nbytes = host.size
        assert nbytes % 256 == 0
        base = torch.from_numpy(host).cuda()
        self.buf = torch.empty((copies, nbytes), dtype=torch.uint8, device="cuda")
        self.buf.copy_(base.unsqueeze(0).expand(copies, nbytes))
        self.tensors = [qh.DeviceTensor(self.buf[i], dtype, rows, cols) for i in range(copies)]


def capture(torch, fn):
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def time_graph(torch, g, steps, warmup):
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3  # seconds


def gemv_rotation(qh, synth, torch, dtype, shapes, steps, warmup, min_bytes=GIB, hot=False, check=None):
    """Times batch-1 GEMVs over a rotation of weight copies. Returns a result dict."""
    per_copy = sum(synth.tensor_bytes(dtype, n, k) for n, k in shapes)
    copies = 1 if hot else max(1, math.ceil(min_bytes / per_copy))
    launches_per_copy = len(shapes)
    reps = 256 if hot else 1  # hot: the same copy many times per step
    rots, acts, outs = [], [], []
    for i, (n, k) in enumerate(shapes):
        host = synth.q8_tensor(100 + i, n, k) if dtype == 2 else synth.q4_tensor(200 + i, n, k)
        rots.append((host, Rotation(qh, torch, host, dtype, n, k, copies)))
        x = torch.from_numpy(synth.activations(300 + i, 1, k)).cuda()
        acts.append(qh.quantize_q8(x[0]))
        outs.append(torch.zeros(n, dtype=torch.float32, device="cuda"))

    def step():
        for _ in range(reps):
            for c in range(copies):
                for (host, rot), (xq, xd), out in zip(rots, acts, outs):
                    qh.matvec_q(rot.tensors[c], xq, xd, out=out)

    g = capture(torch, step)
    sec = time_graph(torch, g, steps, warmup)
    launches = steps * reps * copies * launches_per_copy
    alg = steps * reps * copies * sum(gemv_bytes(dtype, n, k) for n, k in shapes)
    if check is not None:  # the measured path must agree with the oracle, bit for bit
        for (n, k), (host, rot), (xq, xd), out in zip(shapes, rots, acts, outs):
            want = check.matvec_q(dtype, n, k, host, xq.cpu().numpy(), xd.cpu().numpy(), threads=8)
            if not np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32)):
                raise SystemExit(f"bench: GPU GEMV {n}x{k} differs from the oracle")
    del g, rots
    return {"GBps": alg / sec / 1e9, "us_per_launch": sec / launches * 1e6, "launches": launches,
            "bytes_per_launch": alg / launches, "copies": copies, "seconds": sec,
            "ms_per_step": sec / steps * 1e3}


def prefill_rotation(qh, synth, torch, dtype, n, k, m, steps, warmup, min_bytes=GIB // 2):
    wbytes = synth.tensor_bytes(dtype, n, k)
    copies = max(1, math.ceil(min_bytes / wbytes))
    host = synth.q8_tensor(400, n, k) if dtype == 2 else synth.q4_tensor(401, n, k)
    rot = Rotation(qh, torch, host, dtype, n, k, copies)
    x = torch.from_numpy(synth.activations(402, m, k)).cuda()
    xq, xd = qh.quantize_q8(x)
    out = torch.zeros((m, n), dtype=torch.float32, device="cuda")

    def step():
        for c in range(copies):
            qh.matmul_q(rot.tensors[c], xq, xd, out=out)

    g = capture(torch, step)
    sec = time_graph(torch, g, steps, warmup)
    calls = steps * copies
    per = sec / calls
    alg = wbytes + m * 1.125 * k + 4.0 * m * n
    del g, rot
    return {"us_per_call": per * 1e6, "GBps": alg / per / 1e9, "TOPS": 2.0 * m * n * k / per / 1e12,
            "tok_per_s": m / per}


def head_bench(qh, synth, torch, oracle, steps, warmup):
    V, D = 151936, 896
    log("generating the 151936 x 896 head (Q8_0 + Q4_0 copy + bounds)")
    head8, head4, err = synth.shortlist_head(500, V, D)
    per_copy = head8.size + head4.size + err.size * 2
    copies = max(1, math.ceil(GIB / per_copy))
    r8 = Rotation(qh, torch, head8, 2, V, D, copies)
    r4 = Rotation(qh, torch, head4, 3, V, D, copies)
    re = Rotation(qh, torch, err.view(np.uint8).reshape(-1), 1, V, D // 32, copies)
    heads = [qh.ShortlistHead(r8.tensors[c], r4.tensors[c], re.tensors[c], top_k=1) for c in range(copies)]
    n_vec = 8
    x = torch.from_numpy(synth.activations(501, n_vec, D, scale=0.5)).cuda()
    xq, xd = qh.quantize_q8(x)
    # parity of one call against the oracle
    heads[0](xq[0], xd[0])
    st = heads[0].stats()
    o = oracle.shortlist_head(head8, head4, err, V, D, xq[0].cpu().numpy(), xd[0].cpu().numpy(), top_k=1)
    if st["top1"] != oracle.argmax(o["logits"]) or st["n_rows"] != o["n_rows"]:
        raise SystemExit("bench: GPU shortlist head differs from the oracle")
    rows = []
    for t in range(n_vec):
        heads[0](xq[t], xd[t])
        rows.append(heads[0].stats()["n_rows"])
    # rescored rows over 1,024 seeded N(0,1)*0.5 hidden states (check_head's statistics, checks.cpp:178-239)
    n_sweep = 1024
    xs = torch.from_numpy(synth.activations(502, n_sweep, D, scale=0.5)).cuda()
    sq, sd = qh.quantize_q8(xs)
    sweep_rows = []
    for t in range(n_sweep):
        heads[0](sq[t], sd[t])
        sweep_rows.append(heads[0].stats()["n_rows"])
    sweep_rows = np.array(sweep_rows, np.float64)
    del xs, sq, sd

    def sl_step():
        for c in range(copies):
            for t in range(n_vec):
                heads[c](xq[t], xd[t])

    g = capture(torch, sl_step)
    sec = time_graph(torch, g, steps, warmup)
    calls = steps * copies * n_vec
    sl_us = sec / calls * 1e6
    del g
    logits = torch.empty(V, dtype=torch.float32, device="cuda")
    am = qh.Argmax(V)

    def full_step():
        for c in range(copies):
            for t in range(n_vec):
                qh.matvec_q(r8.tensors[c], xq[t], xd[t], out=logits)
                am(logits)

    g = capture(torch, full_step)
    sec = time_graph(torch, g, steps, warmup)
    full_us = sec / calls * 1e6
    del g

    def gemv_step():  # the full head's Q8_0 GEMV alone: the one decode GEMV large enough to stream
        for c in range(copies):
            for t in range(n_vec):
                qh.matvec_q(r8.tensors[c], xq[t], xd[t], out=logits)

    g = capture(torch, gemv_step)
    sec = time_graph(torch, g, steps, warmup)
    gemv_us = sec / calls * 1e6
    gemv_bytes = 1.0625 * V * D + 1.125 * D + 4 * V  # weights and scales, activation, output
    screen = V * (D // 2 + 2 * (D // 32) * 2)
    row8 = D + 2 * (D // 32)
    mean_rows = float(np.mean(rows))
    sl_bytes = screen + mean_rows * row8
    full_bytes = V * row8
    del g, heads, r4, re

    # The nibble-plane head (no Q4_0 copy, no error stream): planes built on the device from the Q8_0 copies, as many
    # as make the screened bytes (high plane + scales) a >= 1 GiB rotation.
    screen_pl = V * (D // 2 + 2 * (D // 32))
    copies_pl = max(1, math.ceil(GIB / screen_pl))
    pls = [qh.head_planes(r8.tensors[c % copies]) for c in range(copies_pl)]
    del r8
    pheads = [qh.ShortlistHead(p, None, None, top_k=1) for p in pls]
    pheads[0](xq[0], xd[0])
    pst = pheads[0].stats()
    po = oracle.shortlist_planes(oracle.head_planes(head8, V, D), V, D, xq[0].cpu().numpy(), xd[0].cpu().numpy(),
                                 top_k=1)
    if pst["top1"] != st["top1"] or pst["n_rows"] != po["n_rows"] or pst["top1"] != oracle.argmax(po["logits"]):
        raise SystemExit("bench: GPU nibble-plane head differs from the oracle")
    p_rows = []
    for t in range(n_vec):
        pheads[0](xq[t], xd[t])
        p_rows.append(pheads[0].stats()["n_rows"])
    xs = torch.from_numpy(synth.activations(502, n_sweep, D, scale=0.5)).cuda()
    sq, sd = qh.quantize_q8(xs)
    p_sweep = []
    for t in range(n_sweep):
        pheads[0](sq[t], sd[t])
        p_sweep.append(pheads[0].stats()["n_rows"])
    p_sweep = np.array(p_sweep, np.float64)
    del xs, sq, sd

    def pl_step():
        for c in range(copies_pl):
            for t in range(n_vec):
                pheads[c](xq[t], xd[t])

    g = capture(torch, pl_step)
    sec = time_graph(torch, g, steps, warmup)
    pl_us = sec / (steps * copies_pl * n_vec) * 1e6
    del g, pheads, pls
    pl_mean = float(np.mean(p_rows))
    pl_bytes = screen_pl + pl_mean * row8
    planes = {"us": pl_us, "mean_rows": pl_mean, "rows": p_rows, "bytes": pl_bytes, "GBps": pl_bytes / pl_us / 1e3,
              "copies": copies_pl, "extra_memory_bytes": 0,
              "sweep_1024": {"vectors": n_sweep, "x_seed": 502, "rows_mean": float(p_sweep.mean()),
                             "rows_median": float(np.median(p_sweep)), "rows_p99": float(np.percentile(p_sweep, 99)),
                             "rows_max": float(p_sweep.max()),
                             "bytes_mean": float((screen_pl + p_sweep * row8).mean()),
                             "bytes_mean_frac_of_full_head": float((screen_pl + p_sweep * row8).mean() / full_bytes)}}
    sweep_bytes = screen + sweep_rows * row8
    return {"shortlist_us": sl_us, "full_head_us": full_us, "mean_rows": mean_rows, "rows": rows,
            "nibble_planes": planes,
            "shortlist_bytes": sl_bytes, "full_head_bytes": full_bytes,
            "shortlist_GBps": sl_bytes / sl_us / 1e3, "full_head_GBps": full_bytes / full_us / 1e3,
            "q8_gemv_151936x896": {"us_per_call": gemv_us, "bytes": gemv_bytes, "GBps": gemv_bytes / gemv_us / 1e3,
                                   "frac_of_hbm_peak": gemv_bytes / gemv_us / 1e3 / HBM_PEAK_GBS},
            "sweep_1024": {"vectors": n_sweep, "x_seed": 502, "rows_mean": float(sweep_rows.mean()),
                           "rows_median": float(np.median(sweep_rows)),
                           "rows_p99": float(np.percentile(sweep_rows, 99)), "rows_max": float(sweep_rows.max()),
                           "rows_mean_frac_of_vocab": float(sweep_rows.mean() / V),
                           "bytes_mean": float(sweep_bytes.mean()),
                           "bytes_mean_frac_of_full_head": float(sweep_bytes.mean() / full_bytes)}}


def sampler_bench(qh, torch, orc, reps=50):
    """One Sampler::sample draw over 151936 device logits (N(0, 3), seed 503; a 64-id history), per parameter set:
    top_k 20 (the one-workgroup kernel), 1000 and 0 (qh_sample_ws: radix sort, then the in-order sums). The first
    draw is checked against the oracle; the time is the mean over `reps` draws captured in one graph."""
    V = 151936
    rng = np.random.default_rng(503)
    host = rng.normal(0.0, 3.0, V).astype(np.float32)
    hist = rng.integers(0, V, 64).astype(np.int32)
    logits = torch.from_numpy(host).cuda()
    hd = torch.from_numpy(hist).cuda()
    ws = qh.sample_workspace(V)
    out = {}
    for name, t in [("topk20_chat", (0.7, 20, 0.8, 0.0, 1.1, 0)), ("topk1000", (1.0, 1000, 0.95, 0.0, 1.1, 0)),
                    ("topk0_topp0.8", (0.7, 0, 0.8, 0.0, 1.1, 0)), ("topk0_topp1", (1.0, 0, 1.0, 0.0, 1.1, 0))]:
        pq, po = qh.qh_sampler_params(*t), orc.SamplerParams(*t)
        st0 = orc.oracle.sampler_seed(7)
        sd = torch.tensor(np.array([st0], np.uint64).view(np.int64), device="cuda")
        got = int(qh.sample(logits, pq, sd, hd, ws=ws).cpu().item())
        want, _, _ = orc.oracle.sample(host, V, hist, po, st0)
        if got != want:
            raise SystemExit(f"bench: sampler draw differs from the oracle ({name})")
        g = capture(torch, lambda: [qh.sample(logits, pq, sd, hd, ws=ws) for _ in range(reps)])
        sec = time_graph(torch, g, 5, 1)
        out[name] = {"us_per_draw": sec / (5 * reps) * 1e6, "params": list(t)}
        del g
    return out


def stage_bytes(hp, pos):
    """Algorithmic bytes of each decode stage of one layer at position pos (weights with their scales, the activation
    and residual rows read and written, the K/V rows attention reads), and of the final norm and shortlist screen."""
    D, F, hd = hp.dim, hp.ffn_dim, hp.head_dim
    qd, kvd = hp.n_heads * hd, hp.n_kv_heads * hd
    q8, q4 = 1 + 2 / 32, 0.5 + 2 / 32
    act = lambda n: n + 4 * n // 32  # noqa: E731  int8 codes + f32 block scales
    return {
        "qkv": (qd + 2 * kvd) * D * q8 + 2 * 4 * D + 4 * (qd + 2 * kvd),
        "attention": 4 * (qd + 2 * kvd) + 2 * 2 * kvd * pos + 2 * 2 * kvd + act(qd),
        "o": D * qd * q8 + act(qd) + 2 * 4 * D,
        "gate_up": 2 * F * D * q4 + 2 * 4 * D + act(F),
        "down": D * F * q4 + act(F) + 2 * 4 * D,
    }


def decode_stages(qh, torch, hp, tens, n_prompt=512, reps=20):
    """Device time of every kernel of a greedy decode step, from position n_prompt on: `reps` steps through
    qh_decoder_step_timed (each kernel launched with start / stop events, the dispatch's own timestamps), each queued
    behind a spin kernel of about 2 ms (torch.cuda._sleep) so the host has enqueued the whole step before the GPU
    reaches it and the kernels run back to back as in a replayed graph. Returns per-stage means over layers and steps
    (kernel time only, the dispatch gaps between kernels excluded), with the algorithmic bytes and the rate they imply,
    and the sum over the step."""
    import ctypes as C
    dec = qh.Decoder(hp, tens, ctx_len=4096)
    ids = np.random.default_rng(9).integers(0, hp.vocab_size, n_prompt).astype(np.int32)
    dec.prefill(ids, 0, top_k=1)
    dec.begin(reps + 2)
    stream = torch.cuda.current_stream()
    cap = 512
    us = np.zeros(cap, np.float32)
    stage = np.zeros(cap, np.int32)
    n = C.c_int32(0)
    kinds = ("qkv", "attention", "o", "gate_up", "down")
    acc, total = {}, 0.0
    torch.cuda.synchronize()
    for rep in range(reps + 1):
        torch.cuda._sleep(4_000_000)
        qh._check(qh.lib().qh_decoder_step_timed(dec.h, 1, C.c_void_p(stream.cuda_stream), us.ctypes.data,
                                                 stage.ctypes.data, cap, C.byref(n)))
        if rep == 0:
            continue  # warm-up
        for i in range(n.value):
            sid = int(stage[i])
            kind = ("final_norm" if sid == qh.STAGE_FINAL_NORM else "head" if sid == qh.STAGE_HEAD else
                    "pick" if sid == qh.STAGE_PICK else kinds[sid % qh.STAGES_PER_LAYER])
            acc.setdefault(kind, []).append(float(us[i]))
            total += float(us[i])
    dec.close()
    pos = n_prompt + reps // 2
    nbytes = stage_bytes(hp, pos)
    out = {"kernels_per_step": int(n.value), "kernel_us_per_step": total / reps, "position": pos}
    for k, v in acc.items():
        per = len(v) / reps  # kernels of this stage per step
        row = {"us_per_kernel": float(np.mean(v)), "kernels_per_step": per}
        if k in nbytes and per == hp.n_layers:
            row["bytes"] = nbytes[k]
            row["GBps"] = nbytes[k] / row["us_per_kernel"] / 1e3
            row["frac_of_hbm_peak"] = row["GBps"] / HBM_PEAK_GBS
        out[k] = row
    return out


def e2e_model():
    import quanta_cpp_amd.qnt as qnt
    hp = qnt.HParams()
    log("generating the synthetic q4mix model (seed 5)")
    return hp, qnt.synthetic_q4mix(5, hp)


SAMPLED_SEED = 0x51A7C0DE


def state_digest(hidden, hq, hd):
    """The end-to-end golden's per-forward fingerprint (tests/golden/make_e2e_golden.py): 8 bytes of the sha256 of the
    final normed hidden state, then 8 of the sha256 of its int8 quantization and block scales, as two uint64."""
    import hashlib
    h1 = hashlib.sha256(np.ascontiguousarray(hidden, np.float32).tobytes()).digest()[:8]
    h2 = hashlib.sha256(np.ascontiguousarray(hq, np.int8).tobytes() +
                        np.ascontiguousarray(hd, np.float32).tobytes()).digest()[:8]
    return np.frombuffer(h1 + h2, np.uint64)


def e2e_bench(qh, torch, hp, tens, steps=256, warmup=3, n_prompt=512, check=True, mode="greedy", head_planes=False):
    """End-to-end generation on the q4mix Qwen2.5-0.5B-shaped model (configuration 5): a 512-token prompt in
    32-token prefill chunks, then `steps` decode steps, each one replay of a HIP graph holding one captured decode step
    (the chosen token is fed back on the device). A warm-up run of `warmup` steps precedes the timed run; the timed
    stream (positions 512 ..) is checked against the reference engine's. mode "greedy": top-1 shortlist queries and
    greedy picks (`quanta gen --greedy`, tests/golden/e2e_q4mix.npz); "chat": the reference's default sampler
    parameters for both the head queries (top-k 20, the whole history as must ids) and the draws (temperature 0.7,
    top-p 0.8, penalty 1.1), seed 0x51A7C0DE (tests/golden/e2e_sampled.npz). head_planes: the tied head as nibble
    planes (no Q4_0 copy or error bounds on the device; the same stream)."""
    dec = qh.Decoder(hp, tens, ctx_len=4096, head_planes=head_planes)
    chat = mode == "chat"
    if chat:
        dec.set_query(qh.sampler_params())
    ids = np.random.default_rng(9).integers(0, hp.vocab_size, n_prompt).astype(np.int32)
    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
    cap = steps + 1
    # warm-up run: prefill, capture the step, a few replays
    if chat:
        dec.set_sampler(qh.sampler_params(), SAMPLED_SEED)
    dec.prefill(ids, 0, top_k=1)
    dec.begin(cap)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            dec.step(top_k=1)
    torch.cuda.current_stream().wait_stream(side)
    for _ in range(min(warmup, steps)):
        graph.replay()
    torch.cuda.synchronize()
    # timed run: prefill, then `steps` replays
    if chat:
        dec.set_sampler(qh.sampler_params(), SAMPLED_SEED)  # the generator restarts from the seed
    e0, e1, e2 = ev(), ev(), ev()
    e0.record()
    dec.prefill(ids, 0, top_k=1)
    e1.record()
    dec.begin(cap)
    torch.cuda.synchronize()
    e2.record()
    for _ in range(steps):
        graph.replay()
    e3 = ev()
    e3.record()
    torch.cuda.synchronize()
    prefill_s = e0.elapsed_time(e1) / 1e3
    decode_s = e2.elapsed_time(e3) / 1e3
    out = dec.outputs(cap)
    status = dec.status()
    # the state after the last timed forward: a digest of the final normed hidden state and its quantization, and the
    # exact logit of the chosen id (a decoder that lands on the same tokens with other states differs here)
    digest = state_digest(dec.hidden(), *dec.hq())
    top_logit = np.float32(dec.stats()["top1_logit"])
    dec.close()
    del graph
    if status:
        raise SystemExit(f"bench: decoder status {status}")
    parity = state_parity = None
    gpath = os.path.join(ROOT, "tests", "golden", "e2e_sampled.npz" if chat else "e2e_q4mix.npz")
    r = {}
    if check and n_prompt == 512 and os.path.exists(gpath):
        g = np.load(gpath, allow_pickle=False)
        want = g["chat_out"] if chat else g["out"]
        n = min(len(want), steps)
        parity = bool((out[:n] == want[:n]).all())
        if not parity:
            raise SystemExit(f"bench: GPU token stream ({mode}) differs from the reference engine's")
        if not chat:
            # state_digests[s] follows forward s (0 = the prefill), top_logit[s] is forward s's chosen logit
            state_parity = bool((digest == g["state_digests"][steps]).all())
            if steps < len(g["top_logit"]):
                state_parity &= bool(top_logit.view(np.uint32) == g["top_logit"][steps].view(np.uint32))
            if not state_parity:
                raise SystemExit(f"bench: GPU decoder state after {steps} steps differs from the reference engine's")
            r["state_equals_reference"] = state_parity
        if chat:  # the GPU head reads the same rows each step (the sampling tests check every step)
            r = {"head_rows_mean": float(np.mean(g["chat_rows"][:n])),
                 "head_rows_fraction": float(np.mean(g["chat_rows"][:n])) / hp.vocab_size}
    return {"prefill_tok_per_s": n_prompt / prefill_s, "prefill_ms": prefill_s * 1e3,
            "decode_tok_per_s": steps / decode_s, "decode_ms_per_token": decode_s / steps * 1e3,
            "stream_equals_reference": parity, "tokens": int(steps), "prompt": int(n_prompt), **r}


def prefill_stack_bench(qh, torch, hp, tens, stacks=(32, 128, 512), reps=5, n_prompt=512):
    """Prefill of the 512-token prompt alone with each prefill stack (qh_decoder_set_prefill_stack: 32 is the
    reference's chunk), best of `reps` runs between HIP events; after each, the final normed state's digest is
    checked against the reference's (tests/golden/e2e_q4mix.npz, forward 0)."""
    ids = np.random.default_rng(9).integers(0, hp.vocab_size, n_prompt).astype(np.int32)
    g = np.load(os.path.join(ROOT, "tests", "golden", "e2e_q4mix.npz"), allow_pickle=False)
    dec = qh.Decoder(hp, tens, ctx_len=4096)
    out = {}
    for st in stacks:
        dec.set_prefill_stack(st)
        best = None
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record()
            dec.prefill(ids, 0, top_k=1)
            e1.record()
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1)
            best = ms if best is None else min(best, ms)
        ok = bool((state_digest(dec.hidden(), *dec.hq()) == g["state_digests"][0]).all())
        if not ok:
            raise SystemExit(f"bench: prefill with stack {st} differs from the reference's state")
        out[f"stack_{st}"] = {"prefill_ms": round(best, 3), "prefill_tok_per_s": round(n_prompt / best * 1e3, 1),
                              "state_equals_reference": ok}
    dec.close()
    return out


def e2e_cpu_sampled(hp, tens, n_prompt=512, n_gen=16):
    """The reference's Session in the chat flow on the host cores (oracle/_ref): the batched prefill then n_gen
    sampled tokens (default SamplerParams for the head queries and the draws), timed as two runs that differ by
    n_gen - 1 decode steps."""
    sys.path.insert(0, ROOT)
    import oracle as orc
    if orc.ref is None:
        return None
    import quanta_cpp_amd.qnt as qnt
    path = os.path.join("/tmp", f"quanta_bench_q4mix_s_{os.getpid()}.qnt")
    qnt.write_qnt(path, hp, tens)
    threads = max(1, min(16, os.cpu_count() or 1))
    try:
        m = orc.ref.load_model(path, 4096, threads)
        ids = np.random.default_rng(9).integers(0, hp.vocab_size, n_prompt).astype(np.int32)
        sp = orc.sampler_params()
        t = []
        for n in (1, n_gen):
            t0 = time.perf_counter()
            orc.ref.gen_sampled(m, ids, n, sp, sp, SAMPLED_SEED)
            t.append(time.perf_counter() - t0)
        orc.ref.free_model(m)
    finally:
        os.remove(path)
    return {"value": (n_gen - 1) / (t[1] - t[0]), "unit": "tok/s", "cores": threads, "kind": "reference",
            "sample": f"reference Session, chat flow: {n_prompt}-token prefill + 1 and + {n_gen} tokens "
                      f"({t[0]:.1f} s, {t[1]:.1f} s), {threads} threads"}


# Host threads one GPU's share of the box allows (the CPU share a one-GPU job gets, whatever os.cpu_count() reports).
BOX_CPU_SHARE = 16


def cpu_model() -> str:
    """The host CPU's model name (what lscpu prints as "Model name"), from /proc/cpuinfo."""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def e2e_cpu_baseline(hp, tens, n_prompt=512, n_gen=16, n_gen_sweep=8):
    """The reference engine itself (oracle/_ref, built from its sources) on the host cores, bounded sample of the same
    workload: Model::forward_batch over the 512-token prompt (32-token chunks) on the box's CPU share, then greedy
    Model::forward decode steps with the Exact Shortlist Head (top_k = 1) at three thread counts, each on the same
    cache: the CPU share (BOX_CPU_SHARE threads, the headline `value`), the reference's default min(8, hardware
    threads / 2) (threadpool.cpp:21-25) and one thread. The model's thread pool is swapped between them
    (ref_model_set_threads)."""
    sys.path.insert(0, ROOT)
    import ctypes as C
    import oracle as orc
    if orc.ref is None:
        return None
    import quanta_cpp_amd.qnt as qnt
    L = orc.ref.lib
    L.ref_model_load.restype = C.c_void_p
    L.ref_model_load.argtypes = [C.c_char_p, C.c_int, C.c_int]
    L.ref_model_free.argtypes = [C.c_void_p]
    L.ref_model_set_threads.argtypes = [C.c_void_p, C.c_int]
    L.ref_model_forward.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p,
                                    C.c_void_p]
    L.ref_model_forward_batch.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p,
                                          C.c_void_p, C.c_void_p]
    hw = os.cpu_count() or 1
    share = max(1, min(BOX_CPU_SHARE, hw))
    default = int(L.ref_default_threads())
    path = os.path.join("/tmp", f"quanta_bench_q4mix_{os.getpid()}.qnt")
    qnt.write_qnt(path, hp, tens)
    sweep = {}
    try:
        m = L.ref_model_load(path.encode(), 4096, share)
        if not m:
            return None
        ids = np.random.default_rng(9).integers(0, hp.vocab_size, n_prompt).astype(np.int32)
        logits = np.zeros(hp.vocab_size, np.float32)
        t0 = time.perf_counter()
        L.ref_model_forward_batch(m, ids.ctypes.data, n_prompt, 0, 1, logits.ctypes.data, None, None, None)
        t1 = time.perf_counter()
        tok = int(np.argmax(logits))
        pos = n_prompt
        for threads, steps in ((share, n_gen), (default, n_gen_sweep), (1, n_gen_sweep)):
            used = L.ref_model_set_threads(m, threads)
            ta = time.perf_counter()
            for _ in range(steps):
                L.ref_model_forward(m, tok, pos, 1, logits.ctypes.data, None, None, None)
                tok = int(np.argmax(logits))
                pos += 1
            sweep[str(used)] = {"decode_tok_per_s": round(steps / (time.perf_counter() - ta), 3), "steps": steps}
        L.ref_model_free(m)
    finally:
        os.remove(path)
    return {"value": sweep[str(share)]["decode_tok_per_s"], "unit": "tok/s", "cores": share, "kind": "reference",
            "prefill_tok_per_s": n_prompt / (t1 - t0), "threads_sweep": sweep, "hardware_concurrency": hw,
            "default_threads": default, "cpu_model": cpu_model(),
            "sample": f"reference engine (oracle/_ref): {n_prompt}-token batched prefill on {share} threads "
                      f"({t1 - t0:.1f} s), then greedy decode steps with the shortlist head from position "
                      f"{n_prompt}: {n_gen} on {share} threads (the value; the CPU share of one GPU of this "
                      f"{hw}-thread host), {n_gen_sweep} on the reference default {default}, {n_gen_sweep} on 1"}


def read_traffic(path):
    """profiles/q4_gemv_traffic.txt: `fetch_bytes_per_launch: X` and `write_bytes_per_launch: Y`."""
    if not os.path.exists(path):
        return None
    vals = {}
    for line in open(path):
        if ":" in line:
            k, v = line.split(":", 1)
            try:
                vals[k.strip()] = float(v.split()[0])
            except (ValueError, IndexError):
                pass
    if "fetch_bytes_per_launch" in vals and "write_bytes_per_launch" in vals:
        return vals["fetch_bytes_per_launch"] + vals["write_bytes_per_launch"]
    return None


def cpu_baseline(synth, shapes, seconds=12.0):
    """The reference's CPU Q4_0 GEMV (or the oracle restatement) on the host cores, bounded sample."""
    sys.path.insert(0, ROOT)
    import oracle as orc
    threads = max(1, min(16, os.cpu_count() or 1))
    hosts = [synth.q4_tensor(200 + i, n, k) for i, (n, k) in enumerate(shapes)]
    xs = [orc.oracle.quantize_q8(synth.activations(300 + i, 1, k)[0]) for i, (n, k) in enumerate(shapes)]
    kind = "reference" if orc.ref is not None else "port"
    total_bytes, total_sec, calls = 0.0, 0.0, 0
    budget = seconds / len(shapes)
    for (n, k), host, (q, d) in zip(shapes, hosts, xs):
        if orc.ref is not None:
            probe = orc.ref.time_matvec_q(3, n, k, host, q, d, threads, 3) / 3
            reps = max(3, int(budget / max(probe, 1e-6)))
            sec = orc.ref.time_matvec_q(3, n, k, host, q, d, threads, reps)
        else:
            t0 = time.perf_counter()
            orc.oracle.matvec_q(3, n, k, host, q, d, threads=threads)
            probe = time.perf_counter() - t0
            reps = max(3, int(budget / max(probe, 1e-6)))
            t0 = time.perf_counter()
            for _ in range(reps):
                orc.oracle.matvec_q(3, n, k, host, q, d, threads=threads)
            sec = time.perf_counter() - t0
        total_bytes += reps * gemv_bytes(3, n, k)
        total_sec += sec
        calls += reps
    return {"value": total_bytes / total_sec / 1e9, "unit": "GB/s", "cores": threads, "kind": kind,
            "sample": f"{calls} Q4_0 GEMV calls (4864x896 and 896x4864, one weight copy each, rows split "
                      f"in chunks of 16 over {threads} threads), {total_sec:.1f} s"}


def e2e_cpu_port(hp, tens, oracle, n_prompt=512, n_gen=4):
    """Fallback when the reference build is absent: the oracle's C restatement of the decoder (single thread),
    prefill of the same prompt, then n_gen greedy steps."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from decoder_util import oracle_decoder
    dec = oracle_decoder(oracle, hp, tens, ctx_len=4096)
    ids = np.random.default_rng(9).integers(0, hp.vocab_size, n_prompt).astype(np.int32)
    t0 = time.perf_counter()
    r = dec.forward_batch(ids, 0, top_k=1)
    t1 = time.perf_counter()
    tok = oracle.argmax(r["logits"])
    for i in range(n_gen):
        r = dec.forward(tok, n_prompt + i, top_k=1)
        tok = oracle.argmax(r["logits"])
    t2 = time.perf_counter()
    return {"value": n_gen / (t2 - t1), "unit": "tok/s", "cores": 1, "kind": "port",
            "prefill_tok_per_s": n_prompt / (t1 - t0),
            "sample": f"oracle C restatement of the decoder, one thread: {n_prompt}-token prefill ({t1 - t0:.1f} s), "
                      f"{n_gen} greedy steps ({t2 - t1:.1f} s)"}


# The reference's published decode rate for this model shape: q4mix-sl, Galaxy S24, best thread count (README.md:35)
BASELINE_DECODE_TOK_S = 78.6


def rnd(d):
    return {k: (round(v, 3) if isinstance(v, float) else v) for k, v in d.items()}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256, help="timed greedy decode steps")
    ap.add_argument("--warmup", type=int, default=3, help="decode steps of the warm-up run")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--e2e-only", action="store_true", help="only the end-to-end prefill + decode measurement")
    ap.add_argument("--stacks", default="32,128,512", help="prefill stacks of --only prefill_stack")
    ap.add_argument("--only", choices=["e2e", "roofline", "prefill", "sampling", "head", "sampler", "stages",
                                       "prefill_stack", "planes"],
                    help="one measurement alone (for counter runs): e2e = --e2e-only; roofline = a 256 MiB copy "
                         "(counter calibration) then the Q4_0 GEMV rotation; prefill = Q4_0 4864x896 and 896x4864 at M = 512, "
                         "then 9728x896 (the decoder's gate + up rows) and 896x4864 (down) at M = 32")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported: this path runs on a single MI355X "
              f"(row-sharding it over several GPUs is a design note, not built)", file=sys.stderr)
        return 2
    import torch
    qh = load_package()
    import quanta_cpp_amd.synth as synth
    sys.path.insert(0, ROOT)
    import oracle as orc
    qh.init(0)
    shapes = [(4864, 896), (896, 4864)]
    if args.only == "roofline":
        src = torch.ones(64 << 20, dtype=torch.float32, device="cuda")  # 256 MiB
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        head = gemv_rotation(qh, synth, torch, 3, shapes, 5, 1, check=orc.oracle)
        print(json.dumps({"calibration_copy_bytes": src.numel() * 4, "q4_gemv": rnd(head)}), flush=True)
        return 0
    if args.only == "prefill":
        out = {"q4_prefill_4864x896_M512": rnd(prefill_rotation(qh, synth, torch, 3, 4864, 896, 512, 5, 1))}
        out["q4_prefill_896x4864_M512"] = rnd(prefill_rotation(qh, synth, torch, 3, 896, 4864, 512, 5, 1))
        out["q4_prefill_9728x896_M32"] = rnd(prefill_rotation(qh, synth, torch, 3, 9728, 896, 32, 5, 1))
        out["q4_prefill_896x4864_M32"] = rnd(prefill_rotation(qh, synth, torch, 3, 896, 4864, 32, 5, 1))
        print(json.dumps(out), flush=True)
        return 0
    if args.only == "head":
        print(json.dumps({"shortlist_head_151936x896": rnd(head_bench(qh, synth, torch, orc.oracle, 5, 1))}),
              flush=True)
        return 0
    if args.only == "planes":
        hp, tens = e2e_model()
        ep = e2e_bench(qh, torch, hp, tens, steps=args.steps, warmup=args.warmup, head_planes=True)
        print(json.dumps({"decode_nibble_planes": rnd(ep)}), flush=True)
        return 0
    if args.only == "sampler":
        print(json.dumps({"sampler_151936": rnd(sampler_bench(qh, torch, orc))}), flush=True)
        return 0
    if args.only == "sampling":
        hp, tens = e2e_model()
        r = e2e_bench(qh, torch, hp, tens, steps=args.steps, warmup=args.warmup, mode="chat")
        print(json.dumps({"sampling_chat": rnd(r)}), flush=True)
        return 0
    if args.only == "prefill_stack":
        hp, tens = e2e_model()
        stacks = tuple(int(x) for x in args.stacks.split(","))
        print(json.dumps({"prefill_stack": prefill_stack_bench(qh, torch, hp, tens, stacks=stacks)}), flush=True)
        return 0
    if args.only == "stages":
        hp, tens = e2e_model()
        print(json.dumps({"decode_stages": decode_stages(qh, torch, hp, tens)}, default=float), flush=True)
        return 0
    if args.only == "e2e":
        args.e2e_only = True
    hp, tens = e2e_model()
    log(f"headline: prefill 512 + {args.steps} greedy decode steps")
    e = e2e_bench(qh, torch, hp, tens, steps=args.steps, warmup=args.warmup)
    if args.e2e_only:
        print(json.dumps(rnd(e)), flush=True)
        return 0
    result = {
        "metric": METRIC, "value": round(e["decode_tok_per_s"], 2), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(e["decode_ms_per_token"], 4),
        "higher_is_better": True, "scaling": "weak",
        "vs_baseline": round(e["decode_tok_per_s"] / BASELINE_DECODE_TOK_S, 2), "dtype": "int8",
        "data": "synthetic random-init q4mix model (seeded, quanta.cpp_amd/qnt.py seed 5; Q8_0 attention, Q4_0 MLP, "
                "Exact Shortlist Head copy), prompt of 512 ids uniform over the vocabulary (seed 9)",
        "config": {"workload": "q4mix Qwen2.5-0.5B-shaped greedy decode (24 layers, dim 896, 14/2 heads, MLP 4864, "
                               "vocab 151936, f16 KV cache, ctx 4096): 512-token prompt in 32-token prefill chunks, "
                               f"then {args.steps} decode steps, one graph-replayed step per token",
                   "prefill_tok_per_s": round(e["prefill_tok_per_s"], 1),
                   "stream_equals_reference": e["stream_equals_reference"],
                   "state_equals_reference": e.get("state_equals_reference"),
                   "head": "Exact Shortlist Head, top_k 1"},
    }
    log("roofline: Q4_0 GEMV at the MLP shapes, cold HBM")
    head = gemv_rotation(qh, synth, torch, 3, shapes, 20, 3, check=orc.oracle)
    achieved = head["bytes_per_launch"] / (head["us_per_launch"] * 1e-6) / 1e9
    traffic = read_traffic(os.path.join(ROOT, "profiles", "q4_gemv_traffic.txt"))
    result["roofline"] = {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                          "kernel": "gemv_kernel<Q4_0> (decode weight GEMV, gate/up 4864x896 + down 896x4864)",
                          "bytes_per_launch": round(head["bytes_per_launch"], 1),
                          "us_per_launch": round(head["us_per_launch"], 3),
                          "copies_per_shape": head["copies"]}
    extra = {"q4_gemv_mlp_GBps": round(head["GBps"], 2)}
    if args.steps != 256:
        log("decode over 256 steps (positions 512-767) beside the timed run's")
        e256 = e2e_bench(qh, torch, hp, tens, steps=256, warmup=args.warmup)
        extra["decode_256_steps"] = {"decode_tok_per_s": round(e256["decode_tok_per_s"], 2),
                                     "decode_ms_per_token": round(e256["decode_ms_per_token"], 4),
                                     "stream_equals_reference": e256["stream_equals_reference"],
                                     "state_equals_reference": e256.get("state_equals_reference")}
    log("decode stages: one traced step per replay")
    st = decode_stages(qh, torch, hp, tens)
    if st is not None:
        nb = stage_bytes(hp, st["position"])
        head_bytes = hp.vocab_size * (hp.dim // 2 + 2 * (hp.dim // 32) * 2) + 200 * (hp.dim + 2 * (hp.dim // 32))
        step_bytes = hp.n_layers * sum(nb.values()) + head_bytes
        extra["decode_stages"] = {k: (rnd(v) if isinstance(v, dict) else v) for k, v in st.items()}
        extra["decode_step_bytes"] = round(step_bytes)
        extra["decode_step_GBps"] = round(step_bytes / (e["decode_ms_per_token"] * 1e-3) / 1e9, 1)
        extra["decode_step_frac_of_hbm_peak"] = round(step_bytes / (e["decode_ms_per_token"] * 1e-3) / 1e9 /
                                                      HBM_PEAK_GBS, 4)
    if not args.no_extra:
        log("Q8_0 / Q4_0 GEMV per shape, cold and hot")
        for dtype, name, shp in [(2, "q8", [(896, 896), (128, 896), (4864, 896), (896, 4864)]),
                                 (3, "q4", shapes)]:
            for n, k in shp:
                cold = gemv_rotation(qh, synth, torch, dtype, [(n, k)], 10, 2)
                hot = gemv_rotation(qh, synth, torch, dtype, [(n, k)], 3, 1, hot=True)
                extra[f"{name}_gemv_{n}x{k}"] = {"cold_GBps": round(cold["GBps"], 1),
                                                  "cold_us": round(cold["us_per_launch"], 3),
                                                  "hot_GBps": round(hot["GBps"], 1),
                                                  "hot_us": round(hot["us_per_launch"], 3)}
        log("prefill matmul")
        for dtype, name, n, k in [(2, "q8", 896, 896), (2, "q8", 128, 896), (3, "q4", 4864, 896),
                                  (3, "q4", 896, 4864)]:
            for m in (32, 128, 512):
                r = prefill_rotation(qh, synth, torch, dtype, n, k, m, 5, 1)
                extra[f"{name}_prefill_{n}x{k}_M{m}"] = rnd(r)
        log("prefill of the 512-token prompt by prefill stack")
        extra["prefill_stack"] = prefill_stack_bench(qh, torch, hp, tens)
        log("shortlist head")
        extra["shortlist_head_151936x896"] = rnd(head_bench(qh, synth, torch, orc.oracle, 5, 1))
        log("greedy decode with the nibble-plane head")
        ep = e2e_bench(qh, torch, hp, tens, steps=args.steps, warmup=args.warmup, head_planes=True)
        extra["decode_nibble_planes"] = {k: (round(v, 3) if isinstance(v, float) else v) for k, v in ep.items()
                                         if k != "prefill_ms"}
        log("sampler draws over the full vocabulary")
        extra["sampler_151936"] = rnd(sampler_bench(qh, torch, orc))
        log("sampling mode: prefill 512 + decode steps of the chat flow")
        extra["sampling_chat"] = rnd(e2e_bench(qh, torch, hp, tens, steps=args.steps, warmup=args.warmup,
                                               mode="chat"))
    result["extra"] = extra
    if not args.no_cpu:
        log("CPU baseline: the reference engine's decoder on the host cores")
        c = e2e_cpu_baseline(hp, tens)
        if c is None:
            c = e2e_cpu_port(hp, tens, orc.oracle)
        result["cpu_baseline"] = rnd(c)
        if not args.no_extra:
            log("CPU baseline: Q4_0 GEMV")
            g = cpu_baseline(synth, shapes)
            extra["q4_gemv_mlp_cpu"] = rnd(g)
            log("CPU baseline: the reference Session in the chat flow")
            extra["sampling_chat_cpu"] = rnd(e2e_cpu_sampled(hp, tens))
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
