"""The one-FMA block product of the eight-wave prefill tile kernel (qh_device.h kSumBias): for an integer block sum s
(|s| <= 32 * 128 * 128 = 2^19) and an f16 row scale d, fma(B + s, d, -(B * d)) with B = 1.5 * 2^23 must be the f32
float(s) * d of ops_ref.cpp:97-98, for every finite f16 d. Checked exactly on the CPU: B + s, B * d and s * d are
exact in float64, so the FMA's single rounding is float32(exact)."""
import numpy as np

B = 12582912.0


def test_bias_bits_are_the_float_sum():
    s = np.arange(-(1 << 19), (1 << 19) + 1, 997, dtype=np.int64)
    biased = (np.int64(0x4B400000) + s).astype(np.uint32).view(np.float32)
    assert (biased.astype(np.float64) == B + s).all()


def test_one_fma_product_equals_float_product_for_every_finite_f16_scale():
    d16 = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    d16 = d16[np.isfinite(d16)]
    d = d16.astype(np.float32)
    cw = -(np.float32(B) * d)  # the staged term, in f32
    assert (cw.astype(np.float64) == -B * d.astype(np.float64)).all(), "-(B * d) is exact"
    rng = np.random.default_rng(0)
    s = np.concatenate([[0, 1, -1, 2, -2, (1 << 19), -(1 << 19), 127 * 127, -127 * 127],
                        rng.integers(-(1 << 19), (1 << 19) + 1, 503)]).astype(np.int64)
    for chunk in np.array_split(s, 8):
        sf = chunk.astype(np.float32)[:, None]
        want = sf * d[None, :]  # float(s) * d, one f32 rounding
        exact = (B + chunk.astype(np.float64))[:, None] * d.astype(np.float64)[None, :] + cw.astype(np.float64)[None, :]
        got = exact.astype(np.float32)  # the FMA's single rounding
        both_zero = (want == 0) & (got == 0)  # the sign of a zero product differs; a chain from +0 never shows it
        assert ((want.view(np.uint32) == got.view(np.uint32)) | both_zero).all()
