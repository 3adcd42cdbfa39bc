#!/usr/bin/env python3
"""Benchmark of the quantized matmul hot path on one MI355X.

Headline workload (one JSON line on stdout): GPTQ-style symmetric 4-bit (Q4_0) decode GEMV, batch 1,
at the Qwen2.5-0.5B MLP shapes gate/up 4864x896 and down 896x4864. A "step" is one pass over a rotation
of distinct weight copies (>= 1 GiB, four times the 256 MB Infinity Cache) so every byte comes from
HBM; the pass is captured once in a HIP graph and replayed. `value` is whole-job algorithmic GB/s:
(0.5625*N*K weight+scale bytes + 1.125*K activation bytes + 4*N output bytes) per GEMV, summed over the
timed steps, divided by the time between two events on the launch stream.

`roofline` covers the same kernel: algorithmic bytes per launch / average launch duration (the timed
region divided by the launch count) against the 8 TB/s HBM peak; `traffic` is the measured HBM bytes
per launch when profiles/q4_gemv_traffic.txt holds rocprofv3 counter readings, else null.
`cpu_baseline` times the reference's own CPU kernel (built from its sources, oracle/_ref) or, where
that build is absent, the oracle's C restatement, on the host cores for a bounded sample.
`extra` adds the other measured configurations: Q8_0 GEMV shapes, hot-cache GEMVs, prefill matmuls at
M = 32/128/512 and the Exact Shortlist Head against the full 8-bit head.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-extra] [--no-cpu]
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
    screen = V * (D // 2 + 2 * (D // 32) * 2)
    row8 = D + 2 * (D // 32)
    mean_rows = float(np.mean(rows))
    sl_bytes = screen + mean_rows * row8
    full_bytes = V * row8
    del g, heads, r8, r4, re
    return {"shortlist_us": sl_us, "full_head_us": full_us, "mean_rows": mean_rows, "rows": rows,
            "shortlist_bytes": sl_bytes, "full_head_bytes": full_bytes,
            "shortlist_GBps": sl_bytes / sl_us / 1e3, "full_head_GBps": full_bytes / full_us / 1e3}


def e2e_model():
    import quanta_cpp_amd.qnt as qnt
    hp = qnt.HParams()
    log("generating the synthetic q4mix model (seed 5)")
    return hp, qnt.synthetic_q4mix(5, hp)


def e2e_bench(qh, torch, hp, tens, steps=256, n_prompt=512, check=True):
    """End-to-end greedy generation on the q4mix Qwen2.5-0.5B-shaped model: prefill of a 512-token prompt in 32-token
    chunks, then `steps` decode steps, each one HIP-graph replay of a captured step (the token is fed back on the
    device). Checks the stream against the reference's (tests/golden/e2e_q4mix.npz) when it is the same workload."""
    dec = qh.Decoder(hp, tens, ctx_len=4096)
    ids = np.random.default_rng(9).integers(0, hp.vocab_size, n_prompt).astype(np.int32)
    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
    dec.prefill(ids, 0, top_k=1)  # warm-up
    torch.cuda.synchronize()
    e0, e1 = ev(), ev()
    e0.record()
    dec.prefill(ids, 0, top_k=1)
    e1.record()
    torch.cuda.synchronize()
    prefill_s = e0.elapsed_time(e1) / 1e3
    dec.begin(steps + 1)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            dec.step(top_k=1)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    e0, e1 = ev(), ev()
    e0.record()
    for _ in range(steps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    decode_s = e0.elapsed_time(e1) / 1e3
    out = dec.outputs(steps + 1)
    parity = None
    gpath = os.path.join(ROOT, "tests", "golden", "e2e_q4mix.npz")
    if check and steps >= 255 and n_prompt == 512 and os.path.exists(gpath):
        g = np.load(gpath, allow_pickle=False)
        parity = bool((out[:256] == g["out"]).all())
        if not parity:
            raise SystemExit("bench: GPU token stream differs from the reference's")
    layer_bytes = sum(_layer_bytes(hp))
    screen_bytes = hp.vocab_size * (hp.dim // 2 + 2 * (hp.dim // 32) * 2)
    dec.close()
    del graph
    return {"prefill_tok_per_s": n_prompt / prefill_s, "prefill_ms": prefill_s * 1e3,
            "decode_tok_per_s": steps / decode_s, "decode_ms_per_token": decode_s / steps * 1e3,
            "decode_weight_GBps": (layer_bytes + screen_bytes) / (decode_s / steps) / 1e9,
            "stream_equals_reference": parity, "tokens": int(steps), "prompt": int(n_prompt)}


def _layer_bytes(hp):
    """Weight bytes one decode step streams through the layers (Q8_0 attention, Q4_0 MLP)."""
    qd, kvd = hp.n_heads * hp.head_dim, hp.n_kv_heads * hp.head_dim
    for _ in range(hp.n_layers):
        yield 1.0625 * (qd * hp.dim + 2 * kvd * hp.dim + hp.dim * qd)
        yield 0.5625 * (3 * hp.ffn_dim * hp.dim)


def e2e_cpu_baseline(hp, tens, n_prompt=64, n_gen=16):
    """The reference engine's own `gen --greedy` flow (oracle/_ref) on the host cores, bounded: a 64-token prompt and
    16 greedy tokens of the same model. Decode rate from the difference of a 16-token and a 1-token run."""
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
    L.ref_gen.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]
    path = os.path.join("/tmp", f"quanta_bench_q4mix_{os.getpid()}.qnt")
    qnt.write_qnt(path, hp, tens)
    threads = max(1, min(16, os.cpu_count() or 1))
    try:
        m = L.ref_model_load(path.encode(), 4096, threads)
        ids = np.random.default_rng(9).integers(0, hp.vocab_size, n_prompt).astype(np.int32)
        out = np.zeros(n_gen, np.int32)
        L.ref_gen(m, ids.ctypes.data, n_prompt, 1, out.ctypes.data, None, None)  # warm-up (page-in)
        t0 = time.perf_counter()
        L.ref_gen(m, ids.ctypes.data, n_prompt, 1, out.ctypes.data, None, None)
        t1 = time.perf_counter()
        L.ref_gen(m, ids.ctypes.data, n_prompt, n_gen, out.ctypes.data, None, None)
        t2 = time.perf_counter()
        L.ref_model_free(m)
    finally:
        os.remove(path)
    one, full = t1 - t0, t2 - t1
    return {"prefill_tok_per_s": n_prompt / one, "decode_tok_per_s": (n_gen - 1) / max(full - one, 1e-9),
            "cores": threads, "kind": "reference",
            "sample": f"reference gen --greedy, {n_prompt}-token prompt, {n_gen} tokens, {threads} threads"}


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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--e2e-only", action="store_true", help="only the end-to-end prefill + decode measurement")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (this path runs on a single "
              f"MI355X; see DESIGN.md for how it would shard)", file=sys.stderr)
        return 2
    import torch
    qh = load_package()
    import quanta_cpp_amd.synth as synth
    sys.path.insert(0, ROOT)
    import oracle as orc
    qh.init(0)
    shapes = [(4864, 896), (896, 4864)]
    if args.e2e_only:
        hp, tens = e2e_model()
        e = e2e_bench(qh, torch, hp, tens, steps=max(args.steps, 256))
        print(json.dumps({kk: (round(v, 3) if isinstance(v, float) else v) for kk, v in e.items()}), flush=True)
        return 0
    log("headline: Q4_0 GEMV rotation")
    head = gemv_rotation(qh, synth, torch, 3, shapes, args.steps, args.warmup, check=orc.oracle)
    result = {
        "metric": METRIC, "value": round(head["GBps"], 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(head["ms_per_step"], 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (seeded: Q4_0 codes uniform [-8,7], scale |N(0,0.02)|/7 per 128 columns; x ~ N(0,1))",
        "config": {"workload": "q4_0 GEMV batch 1, gate/up 4864x896 + down 896x4864, cold HBM rotation",
                   "copies_per_shape": head["copies"], "launches_per_step": head["launches"] // args.steps,
                   "parity": "bit-exact vs oracle"},
    }
    achieved = head["bytes_per_launch"] / (head["us_per_launch"] * 1e-6) / 1e9
    traffic = read_traffic(os.path.join(ROOT, "profiles", "q4_gemv_traffic.txt"))
    result["roofline"] = {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                          "kernel": "gemv_kernel<Q4_0>", "bytes_per_launch": round(head["bytes_per_launch"], 1),
                          "us_per_launch": round(head["us_per_launch"], 3)}
    extra = {}
    if not args.no_extra:
        log("Q8_0 / Q4_0 GEMV per shape, cold and hot")
        for dtype, name, shp in [(2, "q8", [(896, 896), (128, 896), (4864, 896), (896, 4864)]),
                                 (3, "q4", shapes)]:
            for n, k in shp:
                cold = gemv_rotation(qh, synth, torch, dtype, [(n, k)], max(3, args.steps // 2), 2)
                hot = gemv_rotation(qh, synth, torch, dtype, [(n, k)], 3, 1, hot=True)
                extra[f"{name}_gemv_{n}x{k}"] = {"cold_GBps": round(cold["GBps"], 1),
                                                  "cold_us": round(cold["us_per_launch"], 3),
                                                  "hot_GBps": round(hot["GBps"], 1),
                                                  "hot_us": round(hot["us_per_launch"], 3)}
        log("prefill matmul")
        for dtype, name, n, k in [(2, "q8", 896, 896), (2, "q8", 128, 896), (3, "q4", 4864, 896),
                                  (3, "q4", 896, 4864)]:
            for m in (32, 128, 512):
                r = prefill_rotation(qh, synth, torch, dtype, n, k, m, max(3, args.steps // 4), 1)
                extra[f"{name}_prefill_{n}x{k}_M{m}"] = {kk: round(v, 3) for kk, v in r.items()}
        log("shortlist head")
        h = head_bench(qh, synth, torch, orc.oracle, max(3, args.steps // 4), 1)
        extra["shortlist_head_151936x896"] = {kk: (round(v, 3) if isinstance(v, float) else v) for kk, v in h.items()}
        log("end-to-end q4mix decode")
        hp, tens = e2e_model()
        e = e2e_bench(qh, torch, hp, tens)
        extra["e2e_q4mix_qwen2.5_0.5b"] = {kk: (round(v, 3) if isinstance(v, float) else v) for kk, v in e.items()}
    if extra:
        result["extra"] = extra
    if not args.no_cpu:
        log("CPU baseline")
        result["cpu_baseline"] = cpu_baseline(synth, shapes)
        result["cpu_baseline"]["value"] = round(result["cpu_baseline"]["value"], 3)
        if not args.no_extra:
            log("CPU baseline, end to end")
            e = e2e_cpu_baseline(hp, tens)
            if e is not None:
                extra["e2e_q4mix_qwen2.5_0.5b_cpu_reference"] = {kk: (round(v, 3) if isinstance(v, float) else v)
                                                                  for kk, v in e.items()}
                result["extra"] = extra
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
