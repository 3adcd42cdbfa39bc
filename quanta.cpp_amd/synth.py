"""Seeded synthetic tensors in the .qnt block layouts, for parity tests and benchmarks.

Every generator takes a seed and returns numpy arrays whose bytes are exactly what a .qnt file
stores for that tensor (reference scripts/export.py:10-13, engine/src/model_file.h:27-38):

* Q8_0 [rows][cols]: int8 quants [rows*cols] followed by fp16 scales [rows*cols/32];
* Q4_0 [rows][cols]: packed nibbles [rows*cols/2] (per 32-block, byte j holds element j in its
  low nibble and element j+16 in its high nibble, each stored as value+8) followed by fp16 scales.

Distributions follow the benchmark workloads: Q8 codes uniform in [-127, 127] with scales
|N(0, 0.02)|/127; Q4 codes uniform in [-8, 7] with one scale |N(0, 0.02)|/7 per 128 columns,
written into each of its four 32-block scale slots (the format has one scale per 32 weights);
activations N(0, 1). The random stream is numpy's PCG64 (`numpy.random.default_rng(seed)`), and
`digest()` gives a short hash of a buffer so two machines can show they generated the same input.
"""
from __future__ import annotations

import hashlib

import numpy as np

QK = 32
F32, F16, Q8_0, Q4_0 = 0, 1, 2, 3


def quant_bytes(dtype: int, rows: int, cols: int) -> int:
    """Size of the quant section (reference engine/src/model_file.cpp:29-38)."""
    n = rows * cols
    return {F32: 4 * n, F16: 2 * n, Q8_0: n, Q4_0: n // 2}[dtype]


def tensor_bytes(dtype: int, rows: int, cols: int) -> int:
    """Quant section plus the fp16 scale section for quantized types."""
    extra = rows * cols // QK * 2 if dtype in (Q8_0, Q4_0) else 0
    return quant_bytes(dtype, rows, cols) + extra


def digest(*arrays: np.ndarray) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).view(np.uint8).tobytes())
    return h.hexdigest()[:16]


def pack_q4(codes: np.ndarray) -> np.ndarray:
    """int8 codes in [-8, 7], shape [..., cols] -> packed Q4_0 nibbles (uint8, half the size)."""
    nib = (codes.astype(np.int16) + 8).astype(np.uint8).reshape(-1, QK)
    return (nib[:, : QK // 2] | (nib[:, QK // 2 :] << 4)).reshape(-1)


def unpack_q4(packed: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """Inverse of pack_q4: int8 codes [rows][cols]."""
    p = packed[: rows * cols // 2].reshape(-1, QK // 2)
    lo = (p & 15).astype(np.int8) - 8
    hi = (p >> 4).astype(np.int8) - 8
    return np.concatenate([lo, hi], axis=1).reshape(rows, cols)


def q8_tensor(seed: int, rows: int, cols: int) -> np.ndarray:
    """Q8_0 weights: codes uniform [-127, 127], scales f16(|N(0, 0.02)| / 127). Returns uint8 bytes."""
    assert cols % QK == 0
    g = np.random.default_rng(seed)
    q = g.integers(-127, 128, size=rows * cols, dtype=np.int8)
    d = (np.abs(g.standard_normal(rows * cols // QK)) * 0.02 / 127.0).astype(np.float16)
    return np.concatenate([q.view(np.uint8), d.view(np.uint8)])


def q4_tensor(seed: int, rows: int, cols: int, group: int = 128) -> np.ndarray:
    """Q4_0 weights: codes uniform [-8, 7], one f16(|N(0, 0.02)| / 7) per `group` columns replicated into
    each 32-block slot of the group. Returns uint8 bytes."""
    assert cols % group == 0 and group % QK == 0
    g = np.random.default_rng(seed)
    codes = g.integers(-8, 8, size=(rows, cols), dtype=np.int8)
    gs = (np.abs(g.standard_normal(rows * cols // group)) * 0.02 / 7.0).astype(np.float16)
    d = np.repeat(gs, group // QK)
    return np.concatenate([pack_q4(codes), d.view(np.uint8)])


def activations(seed: int, n: int, cols: int, scale: float = 1.0) -> np.ndarray:
    """f32 [n][cols] rows drawn from N(0, scale^2)."""
    g = np.random.default_rng(seed)
    x = g.standard_normal((n, cols))
    if scale != 1.0:
        x = x * scale
    return x.astype(np.float32)


def scales_of(buf: np.ndarray, dtype: int, rows: int, cols: int) -> np.ndarray:
    qb = quant_bytes(dtype, rows, cols)
    return buf[qb : qb + rows * cols // QK * 2].view(np.float16)


def dequant_q8(buf: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """The f32 weights the exact head computes with: code * f16 scale (exact in f32)."""
    q = buf[: rows * cols].view(np.int8).reshape(-1, QK).astype(np.float32)
    d = scales_of(buf, Q8_0, rows, cols).astype(np.float32)
    return (q * d[:, None]).reshape(rows, cols)


def shortlist_copy(head8: np.ndarray, rows: int, cols: int, chunk: int = 4096):
    """Builds the shortlist head's 4-bit copy and its per-block error bound from a Q8_0 head.

    For each 32-block of the dequantized 8-bit head w: the 4-bit scale is the f16 value of
    (signed element of largest magnitude) / -8 times the best of a few stretch factors, the codes are
    round(w / d + 8) clipped to [0, 15], and err is ||w - (code - 8) * d||_2 computed in f64 and rounded
    *up* to f16, so err_b >= the true block error (what the engine's Cauchy-Schwarz bound needs).
    Returns (head4 Q4_0 bytes, err f16 [rows][cols/32])."""
    nb = cols // QK
    packed_parts, scale_parts, err_parts = [], [], []
    for r0 in range(0, rows, chunk):
        r1 = min(rows, r0 + chunk)
        w = dequant_q8(head8_rows(head8, rows, cols, r0, r1), r1 - r0, cols).reshape(-1, QK)
        idx = np.abs(w).argmax(axis=1)
        m = w[np.arange(len(w)), idx]
        best_err = np.full(len(w), np.inf)
        best_d = np.zeros(len(w), np.float16)
        best_q = np.zeros(w.shape, np.uint8)
        for f in (1.0, 0.9, 0.95, 1.05):
            d = (m / -8.0 * f).astype(np.float16)
            df = d.astype(np.float32)
            inv = np.where(df != 0, 1.0 / np.where(df != 0, df, 1), 0).astype(np.float32)
            q = np.clip(np.rint(w * inv[:, None] + 8.0), 0, 15)
            e = (((q - 8.0) * df[:, None] - w) ** 2).sum(axis=1)
            upd = e < best_err
            best_err[upd], best_d[upd], best_q[upd] = e[upd], d[upd], q[upd]
        diff = (best_q.astype(np.float64) - 8.0) * best_d.astype(np.float64)[:, None] - w.astype(np.float64)
        err = np.sqrt((diff * diff).sum(axis=1))
        e16 = err.astype(np.float16)
        low = e16.astype(np.float64) < err
        e16[low] = np.nextafter(e16[low], np.float16(np.inf))
        nib = best_q.astype(np.uint8)
        packed_parts.append(nib[:, : QK // 2] | (nib[:, QK // 2 :] << 4))
        scale_parts.append(best_d)
        err_parts.append(e16)
    head4 = np.concatenate([np.concatenate(packed_parts).reshape(-1), np.concatenate(scale_parts).view(np.uint8)])
    err = np.concatenate(err_parts).reshape(rows, nb)
    return head4, err


def head8_rows(head8: np.ndarray, rows: int, cols: int, r0: int, r1: int) -> np.ndarray:
    """Q8_0 bytes of rows [r0, r1) of a Q8_0 tensor, as a standalone tensor."""
    nb = cols // QK
    q = head8[r0 * cols : r1 * cols]
    s = scales_of(head8, Q8_0, rows, cols)[r0 * nb : r1 * nb]
    return np.concatenate([q, s.view(np.uint8)])


def shortlist_head(seed: int, vocab: int, dim: int):
    """Config-4 head: Q8_0 [vocab][dim] (as q8_tensor) plus its 4-bit copy and error bounds."""
    head8 = q8_tensor(seed, vocab, dim)
    head4, err = shortlist_copy(head8, vocab, dim)
    return head8, head4, err
