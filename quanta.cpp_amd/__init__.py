"""Python binding of libquanta_hip.so (C-ABI in include/quanta_hip.h) for tests and benchmarks.

The directory name is not an importable identifier, so callers load this file by path under the module
name ``quanta_cpp_amd`` (see ``load_package``). Device memory and streams come from torch; every call
goes through the C-ABI into the gfx950 kernels. There is no CPU fallback: if the library is missing or
a call fails, a ``QHError`` is raised.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libquanta_hip.so")
QK = 32
F32, F16, Q8_0, Q4_0 = 0, 1, 2, 3
Q8_0_PLANES = 16  # device-only nibble-plane layout of a Q8_0 head (qh_head_planes)
HEAD_MAX_TOPK = 256
NOALLOC_SCRATCH_BYTES = 4 << 20  # QH_NOALLOC_SCRATCH_BYTES
# status codes (quanta_hip.h)
OK, ERR_ARG, ERR_DTYPE, ERR_SHAPE, ERR_ALIGN, ERR_HIP, ERR_NOMEM, ERR_UNSUPPORTED = range(8)


class QHError(RuntimeError):
    pass


class qh_tensor(C.Structure):
    _fields_ = [("dtype", C.c_int32), ("rows", C.c_int32), ("cols", C.c_int32), ("data", C.c_void_p)]


class qh_head_query(C.Structure):
    _fields_ = [("top_k", C.c_int32), ("n_valid", C.c_int32), ("must", C.c_void_p), ("n_must", C.c_int32)]


class qh_head_stats(C.Structure):
    _fields_ = [("top1", C.c_int32), ("n_rows", C.c_int32), ("n_seeds", C.c_int32), ("n_cand", C.c_int32),
                ("n_must", C.c_int32), ("seed_tie", C.c_int32), ("tau", C.c_float), ("top1_logit", C.c_float)]


class qh_head_out(C.Structure):
    _fields_ = [("logits", C.c_void_p), ("coarse", C.c_void_p), ("upper", C.c_void_p), ("rows", C.c_void_p),
                ("stats", C.c_void_p)]


class qh_model_desc(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("vocab_size", "dim", "n_layers", "n_heads", "n_kv_heads", "head_dim",
                                         "ffn_dim", "ctx_len", "qkv_bias")] + [("rope_theta", C.c_float),
                                                                              ("norm_eps", C.c_float),
                                                                              ("flags", C.c_uint32),
                                                                              ("kv_f32", C.c_int32)]


class qh_decoder_state(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("logits", "hidden", "xq", "xd", "stats", "top1_full", "pos", "n_out",
                                          "token", "kcache", "vcache", "status", "history", "history_len",
                                          "rng_state", "kcache_f32", "vcache_f32")]


class qh_sampler_params(C.Structure):
    """The reference's SamplerParams (sampler.h) without the seed."""
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int32), ("top_p", C.c_float), ("min_p", C.c_float),
                ("repeat_penalty", C.c_float), ("repeat_window", C.c_int32)]


def sampler_params(temperature=0.7, top_k=20, top_p=0.8, min_p=0.0, repeat_penalty=1.1, repeat_window=0):
    """qh_sampler_params with the reference's defaults (sampler.h: Qwen2.5-Instruct's generation config)."""
    return qh_sampler_params(temperature, top_k, top_p, min_p, repeat_penalty, repeat_window)


STAGE_QKV, STAGE_ATTENTION, STAGE_O, STAGE_GATE_UP, STAGE_DOWN, STAGES_PER_LAYER = 0, 1, 2, 3, 4, 8
STAGE_FINAL_NORM, STAGE_HEAD, STAGE_PICK = 1 << 20, (1 << 20) + 1, (1 << 20) + 2

# Every symbol include/quanta_hip.h declares, in header order.
EXPORTS = ("qh_last_error", "qh_version", "qh_init", "qh_quant_bytes", "qh_tensor_bytes", "qh_validate_tensor",
           "qh_malloc", "qh_fault_alloc", "qh_free", "qh_memcpy_h2d", "qh_memcpy_d2h", "qh_memset", "qh_stream_sync",
           "qh_stream_create", "qh_stream_destroy",
           "qh_quantize_q8", "qh_matvec_q", "qh_matvec_ref", "qh_matmul_q", "qh_argmax_workspace_bytes", "qh_argmax",
           "qh_shortlist_workspace_bytes", "qh_shortlist_head", "qh_shortlist_head_noalloc",
           "qh_head_planes", "qh_shortlist_planes",
           "qh_sampler_state", "qh_sample", "qh_sample_workspace_bytes", "qh_sample_ws", "qh_decoder_create",
           "qh_decoder_destroy",
           "qh_decoder_prefill", "qh_decoder_begin", "qh_decoder_step", "qh_decoder_views",
           "qh_decoder_set_prefill_stack", "qh_decoder_step_timed",
           "qh_decoder_set_query",
           "qh_decoder_set_sampler")


def build() -> None:
    """Compile libquanta_hip.so for gfx950 (always recompiles what changed)."""
    subprocess.run(["make", "-s", "-C", HERE, "-j8", "lib"], check=True)


def _bind(lib):
    vp, i32, sz = C.c_void_p, C.c_int, C.c_size_t
    sig = {
        "qh_last_error": ([], C.c_char_p), "qh_version": ([], C.c_char_p), "qh_init": ([i32], i32),
        "qh_quant_bytes": ([i32, i32, i32], sz), "qh_tensor_bytes": ([i32, i32, i32], sz),
        "qh_validate_tensor": ([C.POINTER(qh_tensor)], i32), "qh_malloc": ([C.POINTER(vp), sz], i32),
        "qh_fault_alloc": ([i32], i32),
        "qh_free": ([vp], i32), "qh_memcpy_h2d": ([vp, vp, sz, vp], i32), "qh_memcpy_d2h": ([vp, vp, sz, vp], i32),
        "qh_memset": ([vp, i32, sz, vp], i32), "qh_stream_sync": ([vp], i32),
        "qh_stream_create": ([C.POINTER(vp)], i32), "qh_stream_destroy": ([vp], i32),
        "qh_quantize_q8": ([vp, i32, i32, vp, vp, vp], i32),
        "qh_matvec_q": ([vp, C.POINTER(qh_tensor), vp, vp, i32, i32, vp], i32),
        "qh_matvec_ref": ([vp, C.POINTER(qh_tensor), vp, i32, i32, vp], i32),
        "qh_matmul_q": ([vp, i32, C.POINTER(qh_tensor), vp, vp, i32, i32, i32, vp], i32),
        "qh_argmax_workspace_bytes": ([i32], sz),
        "qh_argmax": ([vp, i32, vp, vp, sz, vp], i32),
        "qh_shortlist_workspace_bytes": ([i32, i32, i32], sz),
        "qh_shortlist_head": ([C.POINTER(qh_tensor)] * 3 + [vp, vp, C.POINTER(qh_head_query), C.POINTER(qh_head_out),
                               vp, sz, vp], i32),
        "qh_shortlist_head_noalloc": ([C.POINTER(qh_tensor)] * 3 + [vp, vp, C.POINTER(qh_head_query),
                                       C.POINTER(qh_head_out), vp], i32),
        "qh_head_planes": ([C.POINTER(qh_tensor), vp, vp], i32),
        "qh_shortlist_planes": ([C.POINTER(qh_tensor), vp, vp, C.POINTER(qh_head_query), C.POINTER(qh_head_out), vp,
                                 sz, vp], i32),
        "qh_decoder_create": ([C.POINTER(qh_model_desc), C.POINTER(qh_tensor), i32, C.POINTER(vp)], i32),
        "qh_decoder_destroy": ([vp], i32),
        "qh_decoder_prefill": ([vp, vp, i32, i32, i32, vp], i32),
        "qh_decoder_begin": ([vp, i32, vp, i32, vp], i32),
        "qh_decoder_step": ([vp, i32, vp], i32),
        "qh_decoder_views": ([vp, C.POINTER(qh_decoder_state)], i32),
        "qh_decoder_set_prefill_stack": ([vp, i32], i32),
        "qh_decoder_step_timed": ([vp, i32, vp, vp, vp, i32, vp], i32),
        "qh_sampler_state": ([C.c_uint64], C.c_uint64),
        "qh_sample": ([vp, i32, vp, vp, vp, i32, C.POINTER(qh_sampler_params), vp, vp, vp], i32),
        "qh_sample_workspace_bytes": ([i32], C.c_size_t),
        "qh_sample_ws": ([vp, i32, vp, vp, vp, i32, C.POINTER(qh_sampler_params), vp, vp, vp, C.c_size_t, vp], i32),
        "qh_decoder_set_query": ([vp, C.POINTER(qh_sampler_params)], i32),
        "qh_decoder_set_sampler": ([vp, C.POINTER(qh_sampler_params), C.c_uint64], i32),
    }
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes, fn.restype = args, res
    return lib


_lib = None


def lib():
    """The loaded library; raises QHError when it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise QHError(f"{LIB_PATH} is missing: build it with `make -C {HERE}` (no CPU fallback exists)")
        _lib = _bind(C.CDLL(LIB_PATH))
    return _lib


def _check(rc: int) -> None:
    if rc != 0:
        raise QHError(f"status {rc}: {lib().qh_last_error().decode()}")


def _torch():
    import torch
    return torch


def _stream():
    return C.c_void_p(_torch().cuda.current_stream().cuda_stream)


def _ptr(t) -> C.c_void_p:
    return C.c_void_p(t.data_ptr())


def init(device: int = 0) -> None:
    _check(lib().qh_init(device))


def tensor_bytes(dtype: int, rows: int, cols: int) -> int:
    return lib().qh_tensor_bytes(dtype, rows, cols)


class DeviceTensor:
    """A .qnt tensor resident in device memory (quants then scales, one allocation)."""

    def __init__(self, buf, dtype: int, rows: int, cols: int):
        self.buf, self.dtype, self.rows, self.cols = buf, dtype, rows, cols
        self.view = qh_tensor(dtype, rows, cols, buf.data_ptr())

    @staticmethod
    def upload(host: np.ndarray, dtype: int, rows: int, cols: int, device="cuda") -> "DeviceTensor":
        torch = _torch()
        host = np.ascontiguousarray(host).view(np.uint8).reshape(-1)
        buf = torch.from_numpy(host.copy()).to(device)
        return DeviceTensor(buf, dtype, rows, cols)

    def validate(self) -> None:
        _check(lib().qh_validate_tensor(C.byref(self.view)))


def quantize_q8(x, q=None, d=None):
    """x: f32 [n_tok][n] (or [n]) device tensor -> (q int8, d f32) device tensors."""
    torch = _torch()
    x2 = x.reshape(-1, x.shape[-1])
    n_tok, n = x2.shape
    if q is None:
        q = torch.empty((n_tok, n), dtype=torch.int8, device=x.device)
    if d is None:
        d = torch.empty((n_tok, n // QK), dtype=torch.float32, device=x.device)
    _check(lib().qh_quantize_q8(_ptr(x2), n_tok, n, _ptr(q), _ptr(d), _stream()))
    shape = x.shape[:-1]
    return q.reshape(*shape, n), d.reshape(*shape, n // QK)


def matvec_q(W: DeviceTensor, xq, xd, out=None, r0: int = 0, r1: int | None = None):
    torch = _torch()
    if out is None:
        out = torch.zeros(W.rows, dtype=torch.float32, device=xq.device)
    r1 = W.rows if r1 is None else r1
    _check(lib().qh_matvec_q(_ptr(out), C.byref(W.view), _ptr(xq), _ptr(xd), r0, r1, _stream()))
    return out


def matvec_ref(W: DeviceTensor, x, out=None, r0: int = 0, r1: int | None = None):
    """W F32 / F16, x [cols] f32 (a device tensor) -> out [rows] with rows [r0, r1) written (matvec_ref)."""
    torch = _torch()
    if out is None:
        out = torch.zeros(W.rows, dtype=torch.float32, device=x.device)
    r1 = W.rows if r1 is None else r1
    _check(lib().qh_matvec_ref(_ptr(out), C.byref(W.view), _ptr(x), r0, r1, _stream()))
    return out


def matmul_q(W: DeviceTensor, xq, xd, out=None, r0: int = 0, r1: int | None = None, ldo: int | None = None):
    """xq [n][cols], xd [n][cols/32] -> out [n][ldo] with rows [r0, r1) written."""
    torch = _torch()
    n = xq.shape[0]
    ldo = W.rows if ldo is None else ldo
    if out is None:
        out = torch.zeros((n, ldo), dtype=torch.float32, device=xq.device)
    r1 = W.rows if r1 is None else r1
    _check(lib().qh_matmul_q(_ptr(out), ldo, C.byref(W.view), _ptr(xq), _ptr(xd), n, r0, r1, _stream()))
    return out


class Argmax:
    """Greedy token of a logits vector of up to `n` entries, with its own workspace."""

    def __init__(self, n: int, device="cuda"):
        torch = _torch()
        self.n = n
        self.ws = torch.empty(lib().qh_argmax_workspace_bytes(n), dtype=torch.uint8, device=device)
        self.index = torch.empty(1, dtype=torch.int32, device=device)

    def __call__(self, logits, n: int | None = None):
        n = logits.numel() if n is None else n
        if n > self.n:
            raise QHError(f"argmax over {n} entries, workspace sized for {self.n}")
        _check(lib().qh_argmax(_ptr(logits), n, _ptr(self.index), _ptr(self.ws), self.ws.numel(), _stream()))
        return self.index


def argmax(logits, n: int | None = None):
    return Argmax(logits.numel(), device=logits.device)(logits, n)


def sampler_state(seed: int) -> int:
    """The generator state a reference Sampler constructed with a nonzero seed starts from."""
    return int(lib().qh_sampler_state(seed))


def sample(logits, params: qh_sampler_params, state, history=None, n_valid: int | None = None, head=None,
           ws=None):
    """One Sampler::sample draw on the device: returns the chosen id as a device int32 tensor of one element.
    state: device uint64 tensor of one element (advanced in place); history: device int32 tensor or None;
    head: a ShortlistHead whose last call's row list and stats restrict the candidates; ws: a device uint8 tensor of
    sample_workspace_bytes(n_valid) bytes for more than SAMPLE_MAX_TOPK survivors (qh_sample_ws), or None."""
    torch = _torch()
    out = torch.empty(1, dtype=torch.int32, device=logits.device)
    nv = logits.numel() if n_valid is None else n_valid
    nh = 0 if history is None else int(history.numel())
    _check(lib().qh_sample_ws(_ptr(logits), nv, _ptr(head.rows) if head is not None else None,
                              _ptr(head.stats_dev) if head is not None else None, _ptr(history) if nh else None, nh,
                              C.byref(params), _ptr(state), _ptr(out), _ptr(ws) if ws is not None else None,
                              0 if ws is None else ws.numel(), _stream()))
    return out


def sample_workspace(n_valid: int, device="cuda"):
    """A device workspace for sample(..., ws=) over n_valid candidates."""
    torch = _torch()
    return torch.empty(int(lib().qh_sample_workspace_bytes(n_valid)), dtype=torch.uint8, device=device)


def head_planes(head8: DeviceTensor) -> DeviceTensor:
    """The nibble-plane layout of a Q8_0 head (qh_head_planes), a new device tensor of the same size."""
    torch = _torch()
    buf = torch.empty(tensor_bytes(Q8_0_PLANES, head8.rows, head8.cols), dtype=torch.uint8, device=head8.buf.device)
    _check(lib().qh_head_planes(C.byref(head8.view), _ptr(buf), _stream()))
    return DeviceTensor(buf, Q8_0_PLANES, head8.rows, head8.cols)


class ShortlistHead:
    """Device-resident Exact Shortlist Head: Q8_0 head, its Q4_0 copy and f16 block error bounds; or a nibble-plane
    head alone (head8 of dtype Q8_0_PLANES, head4 and err None: qh_shortlist_planes)."""

    def __init__(self, head8: DeviceTensor, head4: DeviceTensor | None, err: DeviceTensor | None, top_k: int = 1):
        torch = _torch()
        self.head8, self.head4, self.err = head8, head4, err
        self.V, self.D = head8.rows, head8.cols
        self.top_k = top_k
        nbytes = lib().qh_shortlist_workspace_bytes(self.V, self.D, top_k)
        if nbytes == 0:
            raise QHError(f"unsupported shortlist shape/top_k: {self.V} x {self.D}, k={top_k}")
        dev = head8.buf.device
        self.ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
        self.logits = torch.empty(self.V, dtype=torch.float32, device=dev)
        self.coarse = torch.empty(self.V, dtype=torch.float32, device=dev)
        self.upper = torch.empty(self.V, dtype=torch.float32, device=dev)
        self.stats_dev = torch.zeros(8, dtype=torch.int32, device=dev)
        self._rows_cap = 0
        self.rows = None

    def __call__(self, xq, xd, n_valid: int = 0, must=None, top_k: int | None = None):
        """Enqueues one head call; results stay on the device (see `stats()`)."""
        torch = _torch()
        k = self.top_k if top_k is None else top_k
        if k != self.top_k:
            raise QHError("top_k differs from the one the workspace was sized for")
        n_must = 0 if must is None else int(must.numel())
        if self._rows_cap < self.V + n_must:
            self._rows_cap = self.V + n_must
            self.rows = torch.empty(self._rows_cap, dtype=torch.int32, device=self.logits.device)
        q = qh_head_query(k, n_valid, must.data_ptr() if n_must else None, n_must)
        o = qh_head_out(self.logits.data_ptr(), self.coarse.data_ptr(), self.upper.data_ptr(), self.rows.data_ptr(),
                        self.stats_dev.data_ptr())
        if self.head8.dtype == Q8_0_PLANES:
            _check(lib().qh_shortlist_planes(C.byref(self.head8.view), _ptr(xq), _ptr(xd), C.byref(q), C.byref(o),
                                             _ptr(self.ws), self.ws.numel(), _stream()))
            return
        _check(lib().qh_shortlist_head(C.byref(self.head8.view), C.byref(self.head4.view), C.byref(self.err.view),
                                       _ptr(xq), _ptr(xd), C.byref(q), C.byref(o), _ptr(self.ws),
                                       self.ws.numel(), _stream()))

    def stats(self) -> dict:
        raw = self.stats_dev.cpu().numpy()
        s = qh_head_stats.from_buffer_copy(raw.tobytes())
        return {f: getattr(s, f) for f, _ in qh_head_stats._fields_}


# ------------------------------------------------------------------------------------------------ decoder

LAYER_ORDER = ("input_layernorm.weight", "self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
               "self_attn.o_proj.weight", "self_attn.q_proj.bias", "self_attn.k_proj.bias", "self_attn.v_proj.bias",
               "post_attention_layernorm.weight", "mlp.gate_proj.weight", "mlp.up_proj.weight",
               "mlp.down_proj.weight")


def _d2h(ptr, nbytes, dtype):
    out = np.empty(nbytes // np.dtype(dtype).itemsize, dtype)
    _check(lib().qh_memcpy_d2h(out.ctypes.data, C.c_void_p(ptr), nbytes, _stream()))
    return out


class Decoder:
    """The GPU-resident decoder (qh_decoder_*) over a .qnt tensor set (quanta_cpp_amd.qnt records), uploaded once.
    hp.tied_embeddings false takes lm_head.weight as the LM head, hp.flags carries FLAG_HADAMARD_DOWN, and kv_f32
    keeps an f32 KV cache (Model::load's kv_f16 = false, model.cpp:10, 96-104)."""

    def __init__(self, hp, tensors: dict, ctx_len: int | None = None, device="cuda", kv_f32: bool = False,
                 head_planes: bool = False):
        """head_planes: the Q8_0 LM head (the embedding when tied) is stored as nibble planes (qh_head_planes) in place
        of its Q8_0 form, and the shortlist head screens with the high plane: no head_q4 / head_err are uploaded (the
        scope's nibble-plane variant, zero extra memory)."""
        torch = _torch()
        self.hp = hp
        self.kv_f32 = bool(kv_f32)
        names = ["model.embed_tokens.weight", "model.norm.weight"]
        for l in range(hp.n_layers):
            names += [f"model.layers.{l}.{n}" for n in LAYER_ORDER]
        names += ["quanta.head_q4", "quanta.head_err"]
        tied = getattr(hp, "tied_embeddings", True)
        if not tied:
            names.append("lm_head.weight")
        lm_name = "model.embed_tokens.weight" if tied else "lm_head.weight"
        skip = {"quanta.head_q4", "quanta.head_err"} if head_planes else set()
        if head_planes and tensors[lm_name].dtype != Q8_0:
            raise QHError("head_planes needs a Q8_0 LM head")
        offs, total = [], 0
        for n in names:
            offs.append(total)
            if n in tensors and n not in skip:
                total += (tensors[n].data.size + 255) // 256 * 256
        self.buf = torch.empty(max(total, 256), dtype=torch.uint8, device=device)
        host = np.zeros(max(total, 256), np.uint8)
        for n, o in zip(names, offs):
            if n in tensors and n not in skip and not (head_planes and n == lm_name):
                host[o:o + tensors[n].data.size] = np.asarray(tensors[n].data)
        self.buf.copy_(torch.from_numpy(host))
        del host
        arr = (qh_tensor * len(names))()
        base = self.buf.data_ptr()
        for i, (n, o) in enumerate(zip(names, offs)):
            t = None if n in skip else tensors.get(n)
            arr[i] = qh_tensor(0, 0, 0, None) if t is None else qh_tensor(t.dtype, t.rows, t.cols, base + o)
            if head_planes and n == lm_name:  # the Q8_0 copy goes through a scratch upload into its slot as planes
                q8 = torch.from_numpy(np.ascontiguousarray(t.data).view(np.uint8).reshape(-1)).to(device)
                src = qh_tensor(Q8_0, t.rows, t.cols, q8.data_ptr())
                _check(lib().qh_head_planes(C.byref(src), C.c_void_p(base + o), _stream()))
                torch.cuda.synchronize()
                del q8
                arr[i] = qh_tensor(Q8_0_PLANES, t.rows, t.cols, base + o)
        self._tensors = arr
        self.desc = qh_model_desc(hp.vocab_size, hp.dim, hp.n_layers, hp.n_heads, hp.n_kv_heads, hp.head_dim,
                                  hp.ffn_dim, ctx_len or hp.max_seq, int(hp.qkv_bias), hp.rope_theta, hp.norm_eps,
                                  int(getattr(hp, "flags", 0)), int(self.kv_f32))
        h = C.c_void_p()
        _check(lib().qh_decoder_create(C.byref(self.desc), arr, len(names), C.byref(h)))
        self.h = h
        st = qh_decoder_state()
        _check(lib().qh_decoder_views(self.h, C.byref(st)))
        self.views = st
        self.tokens = None
        self.out = None

    def close(self):
        if getattr(self, "h", None):
            lib().qh_decoder_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_prefill_stack(self, stack: int):
        """Prompt tokens per launch of each layer's norms and matmuls (32 = the reference's chunk; up to 1024), with
        bit-identical results; the device views are re-read (the work buffers move)."""
        _check(lib().qh_decoder_set_prefill_stack(self.h, stack))
        st = qh_decoder_state()
        _check(lib().qh_decoder_views(self.h, C.byref(st)))
        self.views = st

    def prefill(self, tokens, pos0: int = 0, top_k: int = 1):
        torch = _torch()
        self.tokens = torch.as_tensor(np.ascontiguousarray(tokens, np.int32)).to(self.buf.device)
        _check(lib().qh_decoder_prefill(self.h, _ptr(self.tokens), self.tokens.numel(), pos0, top_k, _stream()))

    def begin(self, out_cap: int, top_k: int = 1):
        """Starts a greedy generation into an output list of out_cap tokens. The list's buffer is kept across calls
        with the same capacity, so a decode step captured in a graph after one begin() stays valid after the next."""
        torch = _torch()
        if self.out is None or self.out.numel() != out_cap:
            self.out = torch.zeros(out_cap, dtype=torch.int32, device=self.buf.device)
        else:
            self.out.zero_()
        _check(lib().qh_decoder_begin(self.h, top_k, _ptr(self.out), out_cap, _stream()))

    def step(self, top_k: int = 1):
        _check(lib().qh_decoder_step(self.h, top_k, _stream()))

    def set_query(self, params: qh_sampler_params | None):
        """Head queries as Session::head_query builds them from these sampler parameters (None: plain queries)."""
        self._qp = params
        _check(lib().qh_decoder_set_query(self.h, C.byref(params) if params is not None else None))

    def set_sampler(self, params: qh_sampler_params | None, seed: int = 1):
        """Tokens from Sampler::sample with these parameters and seed (None: the head's greedy top-1)."""
        self._sp = params
        _check(lib().qh_decoder_set_sampler(self.h, C.byref(params) if params is not None else None, seed))

    def history(self):
        """The token history (prompt ids since position 0, then each chosen id)."""
        n = int(_d2h(self.views.history_len, 4, np.int32)[0])
        return _d2h(self.views.history, 4 * n, np.int32) if n else np.zeros(0, np.int32)

    # host copies of the device state (synchronous)
    def stats(self) -> dict:
        raw = _d2h(self.views.stats, C.sizeof(qh_head_stats), np.uint8)
        st = qh_head_stats.from_buffer_copy(raw.tobytes())
        return {f: getattr(st, f) for f, _ in qh_head_stats._fields_}

    def hidden(self):
        return _d2h(self.views.hidden, 4 * self.hp.dim, np.float32)

    def hq(self):
        return _d2h(self.views.xq, self.hp.dim, np.int8), _d2h(self.views.xd, 4 * (self.hp.dim // QK), np.float32)

    def logits(self):
        return _d2h(self.views.logits, 4 * self.hp.vocab_size, np.float32)

    def top1_full(self) -> int:
        return int(_d2h(self.views.top1_full, 4, np.int32)[0])

    def status(self) -> int:
        """0, or bit 0: a step ran past the context (nothing was written); bit 1: a prompt token was out of range."""
        return int(_d2h(self.views.status, 4, np.int32)[0])

    def kv(self, layer: int, n_pos: int):
        """The KV cache of one layer, positions [0, n_pos): (k, v) [n_pos][n_kv_heads*head_dim], as uint16 f16 bits,
        or float32 with kv_f32."""
        kvd = self.hp.n_kv_heads * self.hp.head_dim
        ctx = self.desc.ctx_len
        if self.kv_f32:  # the reference's layout, [ctx][kv_dim] per layer
            off = 4 * layer * ctx * kvd
            return (_d2h(self.views.kcache_f32 + off, 4 * n_pos * kvd, np.float32).reshape(n_pos, kvd),
                    _d2h(self.views.vcache_f32 + off, 4 * n_pos * kvd, np.float32).reshape(n_pos, kvd))
        # K is stored in chunks of 8 dimensions, [n_kv_heads][head_dim / 8][ctx][8]
        rawk = _d2h(self.views.kcache + 2 * layer * ctx * kvd, 2 * ctx * kvd, np.uint16)
        k = np.ascontiguousarray(rawk.reshape(kvd // 8, ctx, 8)[:, :n_pos].transpose(1, 0, 2).reshape(n_pos, kvd))
        # V is stored in blocks of 8 positions, [pos / 8][kv_dim][8]
        nblk = (n_pos + 7) // 8
        raw = _d2h(self.views.vcache + 2 * layer * ((ctx + 7) // 8 * 8) * kvd, 2 * nblk * 8 * kvd, np.uint16)
        v = raw.reshape(nblk, kvd, 8).transpose(0, 2, 1).reshape(nblk * 8, kvd)[:n_pos]
        return k, np.ascontiguousarray(v)

    def position(self) -> int:
        return int(_d2h(self.views.pos, 4, np.int32)[0])

    def outputs(self, n: int):
        return self.out[:n].cpu().numpy()
