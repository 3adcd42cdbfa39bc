"""The .qnt model file: writer, reader, and the synthetic q4mix Qwen2.5-0.5B-shaped model.

Layout (reference engine/src/model_file.cpp:104-218, scripts/export.py:3-13, 291-314), little-endian:
  'QNT1', u32 version (2), hparams: u32 vocab, dim, n_layers, n_heads, n_kv_heads, head_dim, ffn_dim, max_seq,
  f32 rope_theta, f32 norm_eps, u32 tied_embeddings, u32 qkv_bias, u32 flags;
  tokenizer section (u32 length, then: u32 n_tokens + length-prefixed byte strings, u32 n_merges + 3 x u32 each,
  u32 n_specials + (u32 id, string) each, three u32-counted lists of (u32, u32) code-point ranges);
  tensor table: u32 count, then per tensor: string name, u32 dtype, u32 ndim, u32 dims, u64 absolute offset;
  tensor data, each tensor 64-byte aligned. Quantized tensors hold their quants, then fp16 scales per 32 weights.

The synthetic model follows the benchmark's end-to-end configuration: attention projections Q8_0 and MLP projections
4-bit (Q4_0 with one scale per 128 columns written into its four 32-block slots), a tied Q8_0 embedding that is also
the LM head, its shortlist copy (quanta.head_q4, quanta.head_err), norm weights 1.0 and small random q/k/v biases.
Every tensor comes from its own seeded generator (numpy PCG64), so the file is the same on every machine.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass

import numpy as np

from . import synth

MAGIC = b"QNT1"
VERSION = 2
ALIGN = 64
F32, F16, Q8_0, Q4_0 = 0, 1, 2, 3


@dataclass
class HParams:
    vocab_size: int = 151936
    dim: int = 896
    n_layers: int = 24
    n_heads: int = 14
    n_kv_heads: int = 2
    head_dim: int = 64
    ffn_dim: int = 4864
    max_seq: int = 4096
    rope_theta: float = 1e6
    norm_eps: float = 1e-6
    tied_embeddings: bool = True
    qkv_bias: bool = True
    flags: int = 0

    def pack(self) -> bytes:
        return struct.pack("<8I2f3I", self.vocab_size, self.dim, self.n_layers, self.n_heads, self.n_kv_heads,
                           self.head_dim, self.ffn_dim, self.max_seq, self.rope_theta, self.norm_eps,
                           int(self.tied_embeddings), int(self.qkv_bias), self.flags)


@dataclass
class TensorRec:
    dtype: int
    rows: int
    cols: int
    data: np.ndarray  # uint8 bytes as stored in the file
    ndim: int = 2


def _blob(b: bytes) -> bytes:
    return struct.pack("<I", len(b)) + b


def tokenizer_section(n_tokens: int) -> bytes:
    """A byte-level vocabulary: ids 0-255 are the single bytes (the reference tokenizer needs all of them,
    engine/src/tokenizer.cpp:57-61), the others distinct multi-byte strings; no merges, specials or ranges."""
    out = [struct.pack("<I", n_tokens)]
    out += [_blob(bytes([i])) for i in range(min(256, n_tokens))]
    out += [_blob(b"<%d>" % i) for i in range(256, n_tokens)]
    out.append(struct.pack("<I", 0))  # merges
    out.append(struct.pack("<I", 0))  # specials
    out += [struct.pack("<I", 0)] * 3  # letters, numbers, spaces
    return b"".join(out)


def write_qnt(path: str, hp: HParams, tensors: dict[str, TensorRec], n_tokens: int | None = None) -> None:
    names = sorted(tensors)
    tok = tokenizer_section(hp.vocab_size if n_tokens is None else n_tokens)
    head = MAGIC + struct.pack("<I", VERSION) + hp.pack() + _blob(tok)

    def table(offsets):
        t = [struct.pack("<I", len(names))]
        for n in names:
            r = tensors[n]
            dims = (r.cols,) if r.ndim == 1 else (r.rows, r.cols)
            t.append(_blob(n.encode()) + struct.pack("<II", r.dtype, len(dims)) +
                     b"".join(struct.pack("<I", d) for d in dims) + struct.pack("<Q", offsets.get(n, 0)))
        return b"".join(t)

    pos = len(head) + len(table({}))
    offsets = {}
    for n in names:
        pos = (pos + ALIGN - 1) // ALIGN * ALIGN
        offsets[n] = pos
        pos += tensors[n].data.size
    with open(path, "wb") as f:
        f.write(head)
        f.write(table(offsets))
        for n in names:
            f.write(b"\0" * (offsets[n] - f.tell()))
            f.write(np.ascontiguousarray(tensors[n].data).tobytes())


class QntError(ValueError):
    """A .qnt file the reference's loader would refuse; the message is the reference's (model_file.cpp:104-218,
    model.cpp:10-58)."""


class _Cursor:
    """Bounds-checked little-endian reader (model_file.cpp:43-84): reading past the end raises
    'model file truncated'."""

    def __init__(self, buf, p=0, end=None):
        self.buf, self.p, self.end = buf, p, len(buf) if end is None else end

    def need(self, n):
        if self.end - self.p < n:
            raise QntError("model file truncated")

    def take(self, n):
        self.need(n)
        b = self.buf[self.p:self.p + n]
        self.p += n
        return b

    def u32(self):
        return struct.unpack("<I", self.take(4))[0]

    def u64(self):
        return struct.unpack("<Q", self.take(8))[0]

    def f32(self):
        return struct.unpack("<f", self.take(4))[0]

    def str(self):
        return bytes(self.take(self.u32()))

    def ranges(self):
        return [(self.u32(), self.u32()) for _ in range(self.u32())]


def read_qnt(path: str):
    """(HParams, n_tokens, {name: TensorRec}) with tensor data as read-only views into a memory map. Raises QntError
    with the reference reader's message for a file it would refuse (ModelFile::open, model_file.cpp:104-218): bad
    magic or version, a truncated header, tokenizer section or tensor table, a tensor with ndim outside {1, 2}, an
    offset past the end or a tensor running past it. Stricter than the reference in one point: a dtype outside
    F32 / F16 / Q8_0 / Q4_0 is refused here (the reference would size it as 0 bytes)."""
    mm = np.memmap(path, dtype=np.uint8, mode="r")
    buf = memoryview(mm)
    c = _Cursor(buf)
    c.need(4)
    if bytes(c.take(4)) != MAGIC:
        raise QntError("bad magic (not a .qnt file)")
    version = c.u32()
    if version < 1 or version > 2:
        raise QntError(f"unsupported version {version}")
    v = [c.u32() for _ in range(8)]
    rope_theta, norm_eps = c.f32(), c.f32()
    tied, bias = c.u32() != 0, c.u32() != 0
    flags = c.u32() if version >= 2 else 0
    hp = HParams(*v, float(rope_theta), float(norm_eps), tied, bias, flags)
    tok_len = c.u32()
    c.need(tok_len)
    t = _Cursor(buf, c.p, c.p + tok_len)  # the tokenizer section, parsed with its own cursor (model_file.cpp:152-170)
    c.p += tok_len
    n_tokens = t.u32()
    for _ in range(n_tokens):
        t.str()
    for _ in range(t.u32()):
        t.u32(), t.u32(), t.u32()
    for _ in range(t.u32()):
        t.u32(), t.str()
    for _ in range(3):
        t.ranges()
    n_tensors = c.u32()
    tensors = {}
    for _ in range(n_tensors):
        name = c.str().decode(errors="replace")
        dtype, ndim = c.u32(), c.u32()
        if ndim == 1:
            rows, cols = 1, c.u32()
        elif ndim == 2:
            rows, cols = c.u32(), c.u32()
        else:
            raise QntError(f"unsupported ndim for {name}")
        off = c.u64()
        if off > len(mm):
            raise QntError(f"bad offset for {name}")
        if dtype not in (F32, F16, Q8_0, Q4_0):
            raise QntError(f"unsupported dtype {dtype} for {name}")
        size = synth.tensor_bytes(dtype, rows, cols)
        if off + size > len(mm):
            raise QntError(f"tensor out of bounds: {name}")
        if name not in tensors:  # a repeated name keeps its first entry, as the reference's map emplace does
            tensors[name] = TensorRec(dtype, rows, cols, mm[off:off + size], ndim)
    return hp, n_tokens, tensors


FLAG_HADAMARD_DOWN = 1  # model_file.h:21

LAYER_TENSORS = ("input_layernorm.weight", "self_attn.q_proj.weight", "self_attn.k_proj.weight",
                 "self_attn.v_proj.weight", "self_attn.o_proj.weight", "self_attn.q_proj.bias", "self_attn.k_proj.bias",
                 "self_attn.v_proj.bias", "post_attention_layernorm.weight", "mlp.gate_proj.weight",
                 "mlp.up_proj.weight", "mlp.down_proj.weight")


def check_model(hp: HParams, tensors: dict) -> None:
    """Model::load's checks after the file is read (model.cpp:13-58), in its order and with its messages: every tensor
    the forward reads is present (q/k/v biases only with qkv_bias; lm_head.weight only without tied embeddings), the
    Hadamard flag's width rule, the head configuration, and the shortlist tensors' types and shapes."""
    def get(name):
        if name not in tensors:
            raise QntError(f"missing tensor: {name}")
        return tensors[name]

    get("model.embed_tokens.weight")
    get("model.norm.weight")
    lm_head = get("model.embed_tokens.weight") if hp.tied_embeddings else get("lm_head.weight")
    for l in range(hp.n_layers):
        for n in LAYER_TENSORS:
            if n.endswith(".bias") and not hp.qkv_bias:
                continue
            get(f"model.layers.{l}.{n}")
    if (hp.flags & FLAG_HADAMARD_DOWN) and hp.ffn_dim % 256 != 0:
        raise QntError("hadamard flag needs ffn_dim % 256 == 0")
    if hp.n_kv_heads <= 0 or hp.n_heads * hp.head_dim != hp.dim or hp.n_heads % hp.n_kv_heads != 0:
        raise QntError("unsupported head configuration")
    h4, he = tensors.get("quanta.head_q4"), tensors.get("quanta.head_err")
    if h4 is not None or he is not None:
        ok = (h4 is not None and he is not None and h4.dtype == Q4_0 and he.dtype == F16 and lm_head.dtype == Q8_0 and
              h4.rows == lm_head.rows and h4.cols == lm_head.cols and he.rows == lm_head.rows and
              he.cols == lm_head.cols // 32)
        if not ok:
            raise QntError("bad shortlist head tensors")


def load_model(path: str):
    """read_qnt + check_model: (HParams, n_tokens, tensors) of a file the GPU decoder can run, as Model::load
    accepts it; QntError with the reference's message otherwise."""
    hp, n_tokens, tensors = read_qnt(path)
    check_model(hp, tensors)
    return hp, n_tokens, tensors


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, np.float32).view(np.uint8).reshape(-1)


def synthetic_dense(seed: int, hp: HParams | None = None, dtype: int = F32) -> dict[str, TensorRec]:
    """A random-init model stored unquantized, as the exporter writes it with --dtype f32 / f16 (scripts/export.py:211-218:
    every matrix, the embedding included, in that dtype; norms and biases F32): weights N(0, 0.02), rounded to f16 for
    F16; an lm_head.weight of its own with hp.tied_embeddings false; no shortlist tensors (the shortlist head needs a
    Q8_0 LM head, model.cpp:49-58). Sub-seeds: seed * 1000 + a fixed index per tensor."""
    hp = hp or HParams()
    D, F, V = hp.dim, hp.ffn_dim, hp.vocab_size
    qd, kvd = hp.n_heads * hp.head_dim, hp.n_kv_heads * hp.head_dim
    s = lambda i: seed * 1000 + i  # noqa: E731

    def mat(i, rows, cols):
        w = np.random.default_rng(s(i)).standard_normal((rows, cols)).astype(np.float32) * np.float32(0.02)
        if dtype == F16:
            return TensorRec(F16, rows, cols, w.astype(np.float16).view(np.uint8).reshape(-1))
        return TensorRec(F32, rows, cols, _f32(w))

    t: dict[str, TensorRec] = {"model.embed_tokens.weight": mat(0, V, D),
                               "model.norm.weight": TensorRec(F32, 1, D, _f32(np.ones(D)), ndim=1)}
    for l in range(hp.n_layers):
        p = f"model.layers.{l}."
        b = 10 + 20 * l
        t[p + "input_layernorm.weight"] = TensorRec(F32, 1, D, _f32(np.ones(D)), ndim=1)
        t[p + "post_attention_layernorm.weight"] = TensorRec(F32, 1, D, _f32(np.ones(D)), ndim=1)
        t[p + "self_attn.q_proj.weight"] = mat(b + 0, qd, D)
        t[p + "self_attn.k_proj.weight"] = mat(b + 1, kvd, D)
        t[p + "self_attn.v_proj.weight"] = mat(b + 2, kvd, D)
        t[p + "self_attn.o_proj.weight"] = mat(b + 3, D, qd)
        if hp.qkv_bias:
            g = np.random.default_rng(s(b + 4))
            t[p + "self_attn.q_proj.bias"] = TensorRec(F32, 1, qd, _f32(g.standard_normal(qd) * 0.02), ndim=1)
            t[p + "self_attn.k_proj.bias"] = TensorRec(F32, 1, kvd, _f32(g.standard_normal(kvd) * 0.02), ndim=1)
            t[p + "self_attn.v_proj.bias"] = TensorRec(F32, 1, kvd, _f32(g.standard_normal(kvd) * 0.02), ndim=1)
        t[p + "mlp.gate_proj.weight"] = mat(b + 5, F, D)
        t[p + "mlp.up_proj.weight"] = mat(b + 6, F, D)
        t[p + "mlp.down_proj.weight"] = mat(b + 7, D, F)
    if not hp.tied_embeddings:
        t["lm_head.weight"] = mat(1, V, D)
    return t


def synthetic_q4mix(seed: int, hp: HParams | None = None, shortlist: bool = True) -> dict[str, TensorRec]:
    """The random-init q4mix model (tensor name -> record). Sub-seeds: seed * 1000 + a fixed index per tensor. With
    hp.tied_embeddings false an lm_head.weight (Q8_0 [vocab][dim], its own seed) is the LM head, and the shortlist copy
    is made from it; hp.flags (FLAG_HADAMARD_DOWN) changes the forward, not the tensors."""
    hp = hp or HParams()
    D, F, V = hp.dim, hp.ffn_dim, hp.vocab_size
    qd, kvd = hp.n_heads * hp.head_dim, hp.n_kv_heads * hp.head_dim
    s = lambda i: seed * 1000 + i  # noqa: E731
    t: dict[str, TensorRec] = {}
    embed = synth.q8_tensor(s(0), V, D)
    t["model.embed_tokens.weight"] = TensorRec(Q8_0, V, D, embed)
    t["model.norm.weight"] = TensorRec(F32, 1, D, _f32(np.ones(D)), ndim=1)
    for l in range(hp.n_layers):
        p = f"model.layers.{l}."
        b = 10 + 20 * l
        t[p + "input_layernorm.weight"] = TensorRec(F32, 1, D, _f32(np.ones(D)), ndim=1)
        t[p + "post_attention_layernorm.weight"] = TensorRec(F32, 1, D, _f32(np.ones(D)), ndim=1)
        t[p + "self_attn.q_proj.weight"] = TensorRec(Q8_0, qd, D, synth.q8_tensor(s(b + 0), qd, D))
        t[p + "self_attn.k_proj.weight"] = TensorRec(Q8_0, kvd, D, synth.q8_tensor(s(b + 1), kvd, D))
        t[p + "self_attn.v_proj.weight"] = TensorRec(Q8_0, kvd, D, synth.q8_tensor(s(b + 2), kvd, D))
        t[p + "self_attn.o_proj.weight"] = TensorRec(Q8_0, D, qd, synth.q8_tensor(s(b + 3), D, qd))
        if hp.qkv_bias:
            g = np.random.default_rng(s(b + 4))
            t[p + "self_attn.q_proj.bias"] = TensorRec(F32, 1, qd, _f32(g.standard_normal(qd) * 0.02), ndim=1)
            t[p + "self_attn.k_proj.bias"] = TensorRec(F32, 1, kvd, _f32(g.standard_normal(kvd) * 0.02), ndim=1)
            t[p + "self_attn.v_proj.bias"] = TensorRec(F32, 1, kvd, _f32(g.standard_normal(kvd) * 0.02), ndim=1)
        t[p + "mlp.gate_proj.weight"] = TensorRec(Q4_0, F, D, synth.q4_tensor(s(b + 5), F, D))
        t[p + "mlp.up_proj.weight"] = TensorRec(Q4_0, F, D, synth.q4_tensor(s(b + 6), F, D))
        t[p + "mlp.down_proj.weight"] = TensorRec(Q4_0, D, F, synth.q4_tensor(s(b + 7), D, F))
    head = embed
    if not hp.tied_embeddings:
        head = synth.q8_tensor(s(1), V, D)
        t["lm_head.weight"] = TensorRec(Q8_0, V, D, head)
    if shortlist:
        head4, err = synth.shortlist_copy(head, V, D)
        t["quanta.head_q4"] = TensorRec(Q4_0, V, D, head4)
        t["quanta.head_err"] = TensorRec(F16, V, D // 32, err.view(np.uint8).reshape(-1))
    return t
