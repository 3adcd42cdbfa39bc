"""qh_shortlist_head_noalloc (the shortlist head working in the library's own scratch array, no allocation) against
qh_shortlist_head with a caller workspace, through the C-ABI: two calls in a row, the second on a smaller head with
top-k 20 and must ids; every output bit-identical (logits, coarse scores, upper bounds, row list, stats). The size
limit (a head whose workspace exceeds the scratch array is refused before anything is launched) is checked on the host
in test_cpu_abi.py, with no device buffers behind the descriptors."""
import ctypes as C

import numpy as np
import pytest
import torch

from conftest import bits

pytestmark = pytest.mark.gpu


def _upload(qh, synth, V, D, seed):
    head8, head4, err = synth.shortlist_head(seed, V, D)
    return (qh.DeviceTensor.upload(head8, 2, V, D), qh.DeviceTensor.upload(head4, 3, V, D),
            qh.DeviceTensor.upload(err.view(np.uint8), 1, V, D // 32))


def _outputs(V, n_must, dev):
    return {"logits": torch.empty(V, dtype=torch.float32, device=dev),
            "coarse": torch.empty(V, dtype=torch.float32, device=dev),
            "upper": torch.empty(V, dtype=torch.float32, device=dev),
            "rows": torch.empty(V + n_must, dtype=torch.int32, device=dev),
            "stats": torch.zeros(8, dtype=torch.int32, device=dev)}


def _call(qh, heads, xq, xd, top_k, must, ws):
    """One head call through the C-ABI; ws None = the no-allocation entry point."""
    h8, h4, he = heads
    V = h8.rows
    n_must = 0 if must is None else int(must.numel())
    o = _outputs(V, n_must, xq.device)
    q = qh.qh_head_query(top_k, 0, must.data_ptr() if n_must else None, n_must)
    out = qh.qh_head_out(*(o[k].data_ptr() for k in ("logits", "coarse", "upper", "rows", "stats")))
    L = qh.lib()
    args = (C.byref(h8.view), C.byref(h4.view), C.byref(he.view), C.c_void_p(xq.data_ptr()), C.c_void_p(xd.data_ptr()),
            C.byref(q), C.byref(out))
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    if ws is None:
        rc = L.qh_shortlist_head_noalloc(*args, stream)
    else:
        rc = L.qh_shortlist_head(*args, C.c_void_p(ws.data_ptr()), ws.numel(), stream)
    assert rc == 0, L.qh_last_error().decode()
    torch.cuda.synchronize()
    return {k: v.cpu().numpy() for k, v in o.items()}


def _same(a, b):
    sa = qh_stats(a["stats"])
    sb = qh_stats(b["stats"])
    assert sa == sb
    for k in ("logits", "coarse", "upper"):
        assert (bits(a[k]) == bits(b[k])).all(), k
    n, ns, nm = sa["n_rows"], sa["n_seeds"], sa["n_must"]
    ra, rb = a["rows"][:n], b["rows"][:n]
    assert ra[:ns].tolist() == rb[:ns].tolist()  # seeds, best coarse first
    assert ra[n - nm:].tolist() == rb[n - nm:].tolist()  # must ids in query order, last
    assert sorted(ra[ns:n - nm].tolist()) == sorted(rb[ns:n - nm].tolist())  # candidates, unordered


def qh_stats(raw):
    import quanta_cpp_amd as qh
    s = qh.qh_head_stats.from_buffer_copy(np.ascontiguousarray(raw).tobytes())
    return {f: getattr(s, f) for f, _ in qh.qh_head_stats._fields_}


def test_noalloc_equals_workspace_entry(qh, synth, gpu):
    D = 896
    cases = [(151936, 47, 1, None), (20011, 59, 20, [5, 17, 5, 19000, -3, 4000, 123, 17, 20010])]
    for i, (V, seed, top_k, must) in enumerate(cases):
        print(f"noalloc case {i}: V={V} top_k={top_k} must={must is not None}", flush=True)
        heads = _upload(qh, synth, V, D, seed)
        x = torch.from_numpy(synth.activations(seed + 1, 1, D, scale=0.5)).to(gpu)
        xq, xd = qh.quantize_q8(x)
        m = None if must is None else torch.tensor(must, dtype=torch.int32, device=gpu)
        nbytes = qh.lib().qh_shortlist_workspace_bytes(V, D, top_k)
        assert 0 < nbytes <= qh.NOALLOC_SCRATCH_BYTES
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=gpu)
        want = _call(qh, heads, xq[0], xd[0], top_k, m, ws)
        got = _call(qh, heads, xq[0], xd[0], top_k, m, None)
        _same(got, want)
        assert 0 < qh_stats(got["stats"])["n_rows"] < V


def test_noalloc_under_graph_capture(qh, synth, gpu):
    """qh_shortlist_head_noalloc captured in a HIP graph (after the device's first call, which runs qh_init outside
    the capture) and replayed on two different hidden states: each replay equals an eager call on the same input,
    with the program's own eager work between the replays."""
    V, D = 20011, 896
    heads = _upload(qh, synth, V, D, 71)
    h8, h4, he = heads
    xs = torch.from_numpy(synth.activations(72, 3, D, scale=0.5)).to(gpu)
    xq_all, xd_all = qh.quantize_q8(xs)
    xq = xq_all[0].clone()
    xd = xd_all[0].clone()
    must = torch.tensor([7, 19999, 7, 123], dtype=torch.int32, device=gpu)
    _call(qh, heads, xq, xd, 20, must, None)  # first call on the device: qh_init, outside the capture
    o = _outputs(V, int(must.numel()), gpu)
    q = qh.qh_head_query(20, 0, must.data_ptr(), int(must.numel()))
    out = qh.qh_head_out(*(o[k].data_ptr() for k in ("logits", "coarse", "upper", "rows", "stats")))
    L = qh.lib()
    args = (C.byref(h8.view), C.byref(h4.view), C.byref(he.view), C.c_void_p(xq.data_ptr()), C.c_void_p(xd.data_ptr()),
            C.byref(q), C.byref(out))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            rc = L.qh_shortlist_head_noalloc(*args, C.c_void_p(side.cuda_stream))
    torch.cuda.current_stream().wait_stream(side)
    assert rc == 0, L.qh_last_error().decode()
    for r in (1, 2):
        print(f"noalloc graph replay {r}", flush=True)
        xq.copy_(xq_all[r])
        xd.copy_(xd_all[r])
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = {k: v.cpu().numpy() for k, v in o.items()}
        want = _call(qh, heads, xq_all[r], xd_all[r], 20, must, None)
        _same(got, want)
        assert 0 < qh_stats(got["stats"])["n_rows"] < V
    del graph
