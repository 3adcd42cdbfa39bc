"""ctypes bindings of the parity checkers.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's CPU-baseline
leg, as the checker. The product (quanta.cpp_amd) never imports this package.

* `liboracle.so`: the plain-C restatement in quanta_oracle.c (always built by `make -C oracle`).
* `_ref/libquanta_ref.so`: the reference engine's own kernels compiled from its sources plus
  ref_harness.cpp (`make -C oracle ref`, only where the reference tree is mounted). `ref` is None
  when it is absent.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
QK = 32
Q8_0, Q4_0 = 2, 3
# per-layer tensor names in the decoder's order (reference model.cpp:14-33)
LAYER_ORDER = ("input_layernorm.weight", "self_attn.q_proj.weight", "self_attn.k_proj.weight",
               "self_attn.v_proj.weight", "self_attn.o_proj.weight", "self_attn.q_proj.bias", "self_attn.k_proj.bias",
               "self_attn.v_proj.bias", "post_attention_layernorm.weight", "mlp.gate_proj.weight", "mlp.up_proj.weight",
               "mlp.down_proj.weight")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_int, _f = C.c_int, C.c_float


class SamplerParams(C.Structure):
    """qo_sampler_params: the reference's SamplerParams (sampler.h) without the seed."""
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int), ("top_p", C.c_float), ("min_p", C.c_float),
                ("repeat_penalty", C.c_float), ("repeat_window", C.c_int)]


def sampler_params(temperature=0.7, top_k=20, top_p=0.8, min_p=0.0, repeat_penalty=1.1, repeat_window=0):
    """The reference's defaults (sampler.h, Qwen2.5-Instruct's generation config)."""
    return SamplerParams(temperature, top_k, top_p, min_p, repeat_penalty, repeat_window)


def build(ref: bool | None = None) -> None:
    """Compile liboracle.so, and the reference build too when the reference tree is present."""
    subprocess.run(["make", "-s", "-C", HERE, "oracle"], check=True)
    if ref is None:
        ref = os.path.isdir(os.environ.get("REF", "/root/reference") + "/engine/src")
    if ref:
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


def _load(path):
    return C.CDLL(path) if os.path.exists(path) else None


class _Oracle:
    def __init__(self, lib):
        self.lib = lib
        L = lib
        L.qo_fp16_to_f32.argtypes, L.qo_fp16_to_f32.restype = [C.c_uint16], _f
        L.qo_quantize_q8.argtypes = [_f32p, _int, _i8p, _f32p]
        L.qo_matvec_q.argtypes = [_f32p, _int, _int, _int, _u8p, _i8p, _f32p, _int, _int]
        L.qo_matmul_q.argtypes = [_f32p, _int, _int, _int, _int, _u8p, _i8p, _f32p, _int, _int, _int]
        L.qo_matvec_q_mt.argtypes = [_f32p, _int, _int, _int, _u8p, _i8p, _f32p, _int]
        L.qo_matmul_q_mt.argtypes = [_f32p, _int, _int, _int, _int, _u8p, _i8p, _f32p, _int, _int]
        L.qo_argmax.argtypes, L.qo_argmax.restype = [_f32p, _int], _int
        L.qo_shortlist_head.argtypes = [_u8p, _u8p, _u16p, _int, _int, _i8p, _f32p, _int, _int, C.c_void_p, _int,
                                        _f32p, _f32p, _f32p, _i32p, C.POINTER(_int), C.POINTER(_f), C.POINTER(_int)]
        L.qo_shortlist_head.restype = _int
        L.qo_head_planes.argtypes = [_u8p, _int, _int, _u8p]
        L.qo_shortlist_planes.argtypes = [_u8p, _int, _int, _i8p, _f32p, _int, _int, C.c_void_p, _int, _f32p, _f32p,
                                          _f32p, _i32p, C.POINTER(_int), C.POINTER(_f), C.POINTER(_int)]
        L.qo_shortlist_planes.restype = _int

        L.qo_f32_to_f16.argtypes, L.qo_f32_to_f16.restype = [_f], C.c_uint16
        L.qo_decoder_create.argtypes = [_i32p, np.ctypeslib.ndpointer(np.float32), C.c_void_p, _i32p]
        L.qo_decoder_create.restype = C.c_void_p
        L.qo_decoder_free.argtypes = [C.c_void_p]
        L.qo_decoder_kv.argtypes = [C.c_void_p, _int, _int, C.c_void_p, C.c_void_p]
        L.qo_decoder_forward.argtypes = [C.c_void_p, _int, _int, _int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]
        L.qo_decoder_forward_batch.argtypes = [C.c_void_p, _i32p, _int, _int, _int, C.c_void_p, C.c_void_p, C.c_void_p,
                                               C.c_void_p]
        L.qo_rope_table.argtypes = [_f32p, _int, _int, _f]
        L.qo_decoder_set_must.argtypes = [C.c_void_p, C.c_void_p, _int]
        L.qo_sampler_seed.argtypes, L.qo_sampler_seed.restype = [C.c_uint64], C.c_uint64
        L.qo_sample.argtypes = [_f32p, _int, C.c_void_p, _int, C.POINTER(SamplerParams), C.POINTER(C.c_uint64)]
        L.qo_sample.restype = _int

    def fp16_to_f32(self, h: int) -> float:
        return self.lib.qo_fp16_to_f32(h)

    def f32_to_f16(self, f: float) -> int:
        return self.lib.qo_f32_to_f16(f)

    def rope_table(self, n_pos: int, head_dim: int, theta: float) -> np.ndarray:
        cs = np.empty((n_pos, head_dim // 2, 2), np.float32)
        self.lib.qo_rope_table(cs, n_pos, head_dim, theta)
        return cs

    def decoder(self, hp: dict, arrays: list, dtypes: list) -> "Decoder":
        """hp: vocab, dim, n_layers, n_heads, n_kv_heads, head_dim, ffn_dim, ctx_len, qkv_bias, rope_theta, norm_eps;
        arrays / dtypes in the order of qo_decoder_create (None for absent tensors)."""
        return Decoder(self.lib, hp, arrays, dtypes)

    def decoder_for(self, hp, tensors: dict, ctx_len: int | None = None, kv_f32: bool = False) -> "Decoder":
        """The decoder over a .qnt tensor set (name -> record with .data / .dtype, as quanta_cpp_amd.qnt writes and
        reads them) with hyperparameters hp (an HParams record: its flags and tied_embeddings too); kv_f32: an f32 KV
        cache (Model::load with kv_f16 false)."""
        arrays, dtypes = [], []
        names = ["model.embed_tokens.weight", "model.norm.weight"]
        for l in range(hp.n_layers):
            names += [f"model.layers.{l}.{n}" for n in LAYER_ORDER]
        names += ["quanta.head_q4", "quanta.head_err"]
        untied = not getattr(hp, "tied_embeddings", True)
        if untied:
            names.append("lm_head.weight")
        for name in names:
            t = tensors.get(name)
            arrays.append(None if t is None else np.asarray(t.data))
            dtypes.append(-1 if t is None else t.dtype)
        h = dict(vocab=hp.vocab_size, dim=hp.dim, n_layers=hp.n_layers, n_heads=hp.n_heads, n_kv_heads=hp.n_kv_heads,
                 head_dim=hp.head_dim, ffn_dim=hp.ffn_dim, ctx_len=ctx_len or hp.max_seq, qkv_bias=int(hp.qkv_bias),
                 rope_theta=hp.rope_theta, norm_eps=hp.norm_eps, flags=int(getattr(hp, "flags", 0)),
                 kv_f32=int(kv_f32), untied=int(untied))
        return Decoder(self.lib, h, arrays, dtypes)

    def quantize_q8(self, x: np.ndarray):
        x = np.ascontiguousarray(x, np.float32)
        n = x.shape[-1]
        flat = x.reshape(-1, n)
        q = np.empty(flat.shape, np.int8)
        d = np.empty((flat.shape[0], n // QK), np.float32)
        for i in range(flat.shape[0]):
            qi, di = q[i], d[i]
            self.lib.qo_quantize_q8(flat[i], n, qi, di)
        return q.reshape(x.shape), d.reshape(x.shape[:-1] + (n // QK,))

    def matvec_q(self, dtype, rows, cols, buf, xq, xd, r0=0, r1=None, threads=1):
        out = np.zeros(rows, np.float32)
        xq = np.ascontiguousarray(xq, np.int8)
        xd = np.ascontiguousarray(xd, np.float32)
        if threads > 1 and r0 == 0 and r1 is None:
            self.lib.qo_matvec_q_mt(out, dtype, rows, cols, buf, xq, xd, threads)
        else:
            self.lib.qo_matvec_q(out, dtype, rows, cols, buf, xq, xd, r0, rows if r1 is None else r1)
        return out

    def matmul_q(self, dtype, rows, cols, buf, xq, xd, r0=0, r1=None, threads=1):
        xq = np.ascontiguousarray(xq, np.int8)
        xd = np.ascontiguousarray(xd, np.float32)
        n = xq.shape[0]
        out = np.zeros((n, rows), np.float32)
        if threads > 1 and r0 == 0 and r1 is None:
            self.lib.qo_matmul_q_mt(out, rows, dtype, rows, cols, buf, xq, xd, n, threads)
        else:
            self.lib.qo_matmul_q(out, rows, dtype, rows, cols, buf, xq, xd, n, r0, rows if r1 is None else r1)
        return out

    def matvec_f(self, dtype, rows, cols, buf, x, r0=0, r1=None):
        """matvec_ref over F32 / F16 weights (qo_matvec_f)."""
        L = self.lib
        L.qo_matvec_f.argtypes = [_f32p, _int, _int, _int, C.c_void_p, _f32p, _int, _int]
        out = np.zeros(rows, np.float32)
        buf = np.ascontiguousarray(buf)
        L.qo_matvec_f(out, dtype, rows, cols, buf.ctypes.data, np.ascontiguousarray(x, np.float32), r0,
                      rows if r1 is None else r1)
        return out

    def get_row(self, dtype, rows, cols, buf, row):
        L = self.lib
        L.qo_get_row.argtypes = [_f32p, _int, _int, _int, C.c_void_p, _int]
        out = np.zeros(cols, np.float32)
        buf = np.ascontiguousarray(buf)
        L.qo_get_row(out, dtype, rows, cols, buf.ctypes.data, row)
        return out

    def argmax(self, logits: np.ndarray, n: int | None = None) -> int:
        logits = np.ascontiguousarray(logits, np.float32)
        return self.lib.qo_argmax(logits, logits.size if n is None else n)

    def sampler_seed(self, seed: int) -> int:
        return int(self.lib.qo_sampler_seed(seed))

    def sample(self, logits, n_valid, history, params: SamplerParams, state: int):
        """Sampler::sample on a copy of logits; returns (id, penalized logits, next generator state)."""
        lg = np.array(logits, np.float32, copy=True)
        hist = np.ascontiguousarray(history, np.int32)
        st = C.c_uint64(state)
        tid = self.lib.qo_sample(lg, n_valid, hist.ctypes.data if hist.size else None, hist.size, C.byref(params),
                                 C.byref(st))
        return tid, lg, int(st.value)

    def shortlist_head(self, head8, head4, err, V, D, xq, xd, top_k=1, n_valid=0, must=None):
        must_arr = np.ascontiguousarray(must if must is not None else [], np.int32)
        logits = np.empty(V, np.float32)
        coarse = np.empty(V, np.float32)
        upper = np.empty(V, np.float32)
        rows = np.empty(V + must_arr.size, np.int32)
        ns, tau, tie = _int(0), _f(0), _int(0)
        n = self.lib.qo_shortlist_head(head8, head4, np.ascontiguousarray(err).view(np.uint16).reshape(-1), V, D,
                                       np.ascontiguousarray(xq, np.int8), np.ascontiguousarray(xd, np.float32),
                                       top_k, n_valid, must_arr.ctypes.data if must_arr.size else None,
                                       must_arr.size, logits, coarse, upper, rows, C.byref(ns), C.byref(tau),
                                       C.byref(tie))
        return dict(logits=logits, coarse=coarse, upper=upper, rows=rows[:n].copy(), n_rows=n,
                    n_seeds=ns.value, tau=tau.value, seed_tie=bool(tie.value))

    def head_planes(self, head8, V, D):
        """The nibble-plane layout of a Q8_0 [V][D] head (qo_head_planes): uint8 of the Q8_0 tensor's size."""
        head8 = np.ascontiguousarray(head8, np.uint8)
        planes = np.empty(V * D + V * D // 16, np.uint8)
        self.lib.qo_head_planes(head8, V, D, planes)
        return planes

    def shortlist_planes(self, planes, V, D, xq, xd, top_k=1, n_valid=0, must=None):
        """The shortlist head over the nibble planes alone (qo_shortlist_planes); outputs as shortlist_head."""
        must_arr = np.ascontiguousarray(must if must is not None else [], np.int32)
        logits = np.empty(V, np.float32)
        coarse = np.empty(V, np.float32)
        upper = np.empty(V, np.float32)
        rows = np.empty(V + must_arr.size, np.int32)
        ns, tau, tie = _int(0), _f(0), _int(0)
        n = self.lib.qo_shortlist_planes(np.ascontiguousarray(planes, np.uint8), V, D,
                                         np.ascontiguousarray(xq, np.int8), np.ascontiguousarray(xd, np.float32),
                                         top_k, n_valid, must_arr.ctypes.data if must_arr.size else None,
                                         must_arr.size, logits, coarse, upper, rows, C.byref(ns), C.byref(tau),
                                         C.byref(tie))
        return dict(logits=logits, coarse=coarse, upper=upper, rows=rows[:n].copy(), n_rows=n,
                    n_seeds=ns.value, tau=tau.value, seed_tie=bool(tie.value))


class Decoder:
    """The oracle's decoder (qo_decoder_*): the reference's Model::forward / forward_batch restated in C."""

    def __init__(self, lib, hp, arrays, dtypes):
        self.lib = lib
        self.V, self.D = hp["vocab"], hp["dim"]
        self._keep = [None if a is None else np.ascontiguousarray(a) for a in arrays]
        self._ptrs = (C.c_void_p * len(arrays))(*[None if a is None else a.ctypes.data for a in self._keep])
        hp = dict(hp)
        hp.setdefault("flags", 0)
        hp.setdefault("kv_f32", 0)
        hp.setdefault("untied", 0)
        self.kv_f32 = bool(hp["kv_f32"])
        ints = np.array([hp[k] for k in ("vocab", "dim", "n_layers", "n_heads", "n_kv_heads", "head_dim", "ffn_dim",
                                         "ctx_len", "qkv_bias", "flags", "kv_f32", "untied")], np.int32)
        floats = np.array([hp["rope_theta"], hp["norm_eps"]], np.float32)
        self._dt = np.array(dtypes, np.int32)
        self.h = lib.qo_decoder_create(ints, floats, C.cast(self._ptrs, C.c_void_p), self._dt)
        if not self.h:
            raise ValueError("qo_decoder_create rejected the model")

    def __del__(self):
        if getattr(self, "h", None):
            self.lib.qo_decoder_free(self.h)
            self.h = None

    def _outs(self):
        return (np.empty(self.V, np.float32), np.empty(self.D, np.float32), np.empty(self.D, np.int8),
                np.empty(self.D // QK, np.float32))

    def set_must(self, must):
        """Must ids of the following head queries (None for none)."""
        self._must = None if must is None else np.ascontiguousarray(must, np.int32)
        n = 0 if self._must is None else self._must.size
        self.lib.qo_decoder_set_must(self.h, self._must.ctypes.data if n else None, n)

    def forward(self, token, pos, top_k=1):
        lg, h, q, d = self._outs()
        rows = self.lib.qo_decoder_forward(self.h, token, pos, top_k, lg.ctypes.data, h.ctypes.data, q.ctypes.data,
                                           d.ctypes.data)
        return dict(logits=lg, hidden=h, hq=q, hd=d, rows=rows)

    def kv(self, layer, n_pos, kv_dim):
        """The KV cache of one layer, positions [0, n_pos): (k, v) as [n_pos][kv_dim] f16 bits (uint16), or f32 values
        with an f32 cache."""
        dt = np.float32 if self.kv_f32 else np.uint16
        k = np.empty((n_pos, kv_dim), dt)
        v = np.empty((n_pos, kv_dim), dt)
        self.lib.qo_decoder_kv(self.h, layer, n_pos, k.ctypes.data, v.ctypes.data)
        return k, v

    def forward_batch(self, tokens, pos0, top_k=1):
        lg, h, q, d = self._outs()
        tokens = np.ascontiguousarray(tokens, np.int32)
        rows = self.lib.qo_decoder_forward_batch(self.h, tokens, tokens.size, pos0, top_k, lg.ctypes.data,
                                                 h.ctypes.data, q.ctypes.data, d.ctypes.data)
        return dict(logits=lg, hidden=h, hq=q, hd=d, rows=rows)


class _Ref:
    """The reference engine's own kernels (compiled from its sources)."""

    def __init__(self, lib):
        self.lib = L = lib
        L.ref_fp16_to_f32.argtypes, L.ref_fp16_to_f32.restype = [C.c_uint16], _f
        L.ref_quantize_q8.argtypes = [_f32p, _int, _i8p, _f32p]
        L.ref_matvec_q.argtypes = [_f32p, _int, _int, _int, _u8p, _i8p, _f32p, _int]
        L.ref_matmul_q.argtypes = [_f32p, _int, _int, _int, _u8p, _i8p, _f32p, _int, _int]
        L.ref_shortlist_head.argtypes = [_u8p, _u8p, _u16p, _int, _int, _i8p, _f32p, _int, _int, C.c_void_p, _int,
                                         _int, _f32p, _f32p, _f32p, _i32p]
        L.ref_shortlist_head.restype = _int
        L.ref_time_matvec_q.argtypes = [_f32p, _int, _int, _int, _u8p, _i8p, _f32p, _int, _int]
        L.ref_time_matvec_q.restype = C.c_double
        L.ref_sample.argtypes = [_f32p, _int, C.c_void_p, _int, _f, _int, _f, _f, _f, _int, C.POINTER(C.c_uint64)]
        L.ref_sample.restype = _int
        L.ref_model_load.argtypes, L.ref_model_load.restype = [C.c_char_p, _int, _int], C.c_void_p
        L.ref_model_free.argtypes = [C.c_void_p]
        L.ref_gen_sampled.argtypes = [C.c_void_p, _i32p, _int, _int, _f, _int, _f, _int, _f, _int, _f, _f, _f, _int,
                                      C.c_uint64, _i32p, _i32p]
        L.ref_gen_sampled.restype = _int

    def sample(self, logits, n_valid, history, params: SamplerParams, state: int):
        """The reference's Sampler::sample on a copy of logits: (id, penalized logits, next generator state)."""
        lg = np.array(logits, np.float32, copy=True)
        hist = np.ascontiguousarray(history, np.int32)
        st = C.c_uint64(state)
        tid = self.lib.ref_sample(lg, n_valid, hist.ctypes.data if hist.size else None, hist.size, params.temperature,
                                  params.top_k, params.top_p, params.min_p, params.repeat_penalty,
                                  params.repeat_window, C.byref(st))
        return tid, lg, int(st.value)

    def load_error(self, path: str):
        """The reference Model::load's verdict on a file: None if it loads, else its error message."""
        L = self.lib
        L.ref_model_load_error.argtypes, L.ref_model_load_error.restype = [C.c_char_p, C.c_char_p, _int], _int
        buf = C.create_string_buffer(512)
        return None if L.ref_model_load_error(path.encode(), buf, 512) else buf.value.decode()

    def load_model(self, path: str, ctx_len: int, threads: int, kv_f16: bool = True):
        L = self.lib
        L.ref_model_load_kv.argtypes, L.ref_model_load_kv.restype = [C.c_char_p, _int, _int, _int], C.c_void_p
        m = L.ref_model_load_kv(path.encode(), ctx_len, threads, int(kv_f16))
        if not m:
            raise ValueError(f"the reference could not load {path}")
        return m

    def free_model(self, m):
        self.lib.ref_model_free(m)

    def gen_sampled(self, m, ids, n_gen, query: SamplerParams, sampler: SamplerParams, seed: int):
        """A batched-prefill Session whose head queries follow `query` and whose tokens come from
        Sampler(sampler, seed): (ids, per-step head rows)."""
        ids = np.ascontiguousarray(ids, np.int32)
        out = np.zeros(n_gen, np.int32)
        rows = np.zeros(n_gen, np.int32)
        n = self.lib.ref_gen_sampled(m, ids, ids.size, n_gen, query.temperature, query.top_k, query.repeat_penalty,
                                     query.repeat_window, sampler.temperature, sampler.top_k, sampler.top_p,
                                     sampler.min_p, sampler.repeat_penalty, sampler.repeat_window, seed, out, rows)
        if n < 0:
            raise ValueError("prompt does not fit the context")
        return out[:n], rows[:n]

    def fp16_to_f32(self, h: int) -> float:
        return self.lib.ref_fp16_to_f32(h)

    def quantize_q8(self, x: np.ndarray):
        x = np.ascontiguousarray(x, np.float32)
        n = x.shape[-1]
        q = np.empty(n, np.int8)
        d = np.empty(n // QK, np.float32)
        self.lib.ref_quantize_q8(x, n, q, d)
        return q, d

    def matvec_q(self, dtype, rows, cols, buf, xq, xd, threads=1):
        out = np.zeros(rows, np.float32)
        self.lib.ref_matvec_q(out, dtype, rows, cols, buf, np.ascontiguousarray(xq, np.int8),
                              np.ascontiguousarray(xd, np.float32), threads)
        return out

    def time_matvec_q(self, dtype, rows, cols, buf, xq, xd, threads, reps):
        """Seconds for `reps` row-parallel matvec calls on one reference thread pool."""
        out = np.zeros(rows, np.float32)
        return self.lib.ref_time_matvec_q(out, dtype, rows, cols, buf, np.ascontiguousarray(xq, np.int8),
                                          np.ascontiguousarray(xd, np.float32), threads, reps)

    def matvec_f(self, dtype, rows, cols, buf, x, threads=1):
        """Model::linear for an F32 / F16 W (matvec_ref)."""
        L = self.lib
        L.ref_matvec_f.argtypes = [_f32p, _int, _int, _int, _u8p, _f32p, _int]
        out = np.zeros(rows, np.float32)
        L.ref_matvec_f(out, dtype, rows, cols, np.ascontiguousarray(buf).view(np.uint8).reshape(-1),
                       np.ascontiguousarray(x, np.float32), threads)
        return out

    def get_row(self, dtype, rows, cols, buf, row):
        L = self.lib
        L.ref_get_row.argtypes = [_f32p, _int, _int, _int, _u8p, _int]
        out = np.zeros(cols, np.float32)
        L.ref_get_row(out, dtype, rows, cols, np.ascontiguousarray(buf).view(np.uint8).reshape(-1), row)
        return out

    def matmul_q(self, dtype, rows, cols, buf, xq, xd, threads=1):
        xq = np.ascontiguousarray(xq, np.int8)
        n = xq.shape[0]
        out = np.zeros((n, rows), np.float32)
        self.lib.ref_matmul_q(out, dtype, rows, cols, buf, xq, np.ascontiguousarray(xd, np.float32), n, threads)
        return out

    def shortlist_head(self, head8, head4, err, V, D, xq, xd, top_k=1, n_valid=0, must=None, threads=1):
        must_arr = np.ascontiguousarray(must if must is not None else [], np.int32)
        logits = np.empty(V, np.float32)
        coarse = np.empty(V, np.float32)
        upper = np.empty(V, np.float32)
        rows = np.empty(V + must_arr.size, np.int32)
        n = self.lib.ref_shortlist_head(head8, head4, np.ascontiguousarray(err).view(np.uint16).reshape(-1), V, D,
                                        np.ascontiguousarray(xq, np.int8), np.ascontiguousarray(xd, np.float32),
                                        top_k, n_valid, must_arr.ctypes.data if must_arr.size else None,
                                        must_arr.size, threads, logits, coarse, upper, rows)
        return dict(logits=logits, coarse=coarse, upper=upper, rows=rows[:n].copy(), n_rows=n)


_olib = _load(os.path.join(HERE, "liboracle.so"))
oracle = _Oracle(_olib) if _olib is not None else None
_rlib = _load(os.path.join(HERE, "_ref", "libquanta_ref.so"))
ref = _Ref(_rlib) if _rlib is not None else None
