"""Inputs of the reference's model-free kernel self-test, regenerated from its recipe.

engine/src/checks.cpp:64-87 and :116-120 draw everything from one xorshift64 stream (shifts 13, 7, 17;
seed 0x9E3779B97F4A7C15) in this order, per dtype (Q8_0 first, then Q4_0, the stream continuing):
  quant bytes    uint8(r)                     rows*cols (Q8_0) or rows*cols/2 (Q4_0) values
  fp16 scales    0x2000 + r % 0x800           rows*cols/32 values
  activation     (int(r % 2001) - 1000) / 1000.f, 896 values
  32 activations the same, 32 x 896 values (the prefill tokens)
The shape is one Qwen2.5-0.5B MLP matrix, 4864 x 896. The returned buffers are the .qnt bytes of W
(quants, then scales) and the f32 activations before quantization.
"""
import numpy as np

ROWS, COLS, QK = 4864, 896, 32
SEED = 0x9E3779B97F4A7C15
_M64 = (1 << 64) - 1


def _stream(state, n):
    """n successive xorshift64 outputs as uint64, and the final state."""
    out = np.empty(n, np.uint64)
    s = state
    for i in range(n):
        s ^= (s << 13) & _M64
        s ^= s >> 7
        s ^= (s << 17) & _M64
        out[i] = s
    return out, s


def _acts(r):
    return ((r % np.uint64(2001)).astype(np.int64) - 1000).astype(np.float32) / np.float32(1000.0)


_cache = None


def selftest_inputs():
    """[(dtype, name, {"w": uint8 bytes, "x": f32 [896], "xs": f32 [32][896]})] for Q8_0 then Q4_0."""
    global _cache
    if _cache is not None:
        return _cache
    state = SEED
    res = []
    for dtype, name in ((2, "q8"), (3, "q4")):
        qbytes = ROWS * COLS if dtype == 2 else ROWS * COLS // 2
        nsc = ROWS * COLS // QK
        r, state = _stream(state, qbytes + nsc + COLS + 32 * COLS)
        q = (r[:qbytes] & np.uint64(0xFF)).astype(np.uint8)
        sc = (np.uint64(0x2000) + r[qbytes:qbytes + nsc] % np.uint64(0x800)).astype(np.uint16)
        x = _acts(r[qbytes + nsc:qbytes + nsc + COLS])
        xs = _acts(r[qbytes + nsc + COLS:]).reshape(32, COLS)
        res.append((dtype, name, {"w": np.concatenate([q, sc.view(np.uint8)]), "x": x, "xs": xs}))
    _cache = res
    return res
