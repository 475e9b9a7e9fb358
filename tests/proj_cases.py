"""GGUF weight rows for the projection tests: random payload bytes with fp16
scale fields set to finite values of a realistic size (a row of uniform
random bytes would mostly hold scales of 1e4 and NaNs), plus rows with the
special scale codes a quantizer can write (0, -0, subnormal, negative)."""
import numpy as np

import oracle as O

# byte offsets of the fp16 scale fields inside one block (cpp/quant.hpp:33-63)
SCALE_FIELDS = {O.GGUF_Q4_0: (0,), O.GGUF_Q8_0: (0,), O.GGUF_Q4_K: (0, 2), O.GGUF_Q6_K: (208,)}
# scale ranges that keep |w| at most about 0.2, as in trained models (the
# integer sub-scales and quants multiply them: Q4_0 8, Q8_0 128, Q4_K 63 * 15,
# Q6_K 127 * 32)
SCALE_RANGE = {O.GGUF_Q4_0: (1e-3, 2e-2), O.GGUF_Q8_0: (1e-4, 1.5e-3), O.GGUF_Q4_K: (1e-5, 2e-4),
               O.GGUF_Q6_K: (1e-6, 5e-5)}
SPECIAL_F16 = np.array([0x0000, 0x8000, 0x0001, 0x03FF, 0x8123, 0xBC00], np.uint16)  # 0, -0, subnormals, -1


def make_rows(rng, wtype, rows, n, special=False):
    """uint8 [rows][row bytes] of type wtype for rows of n elements."""
    be, bb = O.GGUF_BLOCK[wtype]
    nb = n // be
    if wtype == O.GGUF_F32:
        return (rng.standard_normal((rows, n)) * 0.05).astype("<f4").view(np.uint8).reshape(rows, -1)
    if wtype == O.GGUF_F16:
        return (rng.standard_normal((rows, n)) * 0.05).astype("<f2").view(np.uint8).reshape(rows, -1)
    raw = rng.integers(0, 256, (rows, nb, bb), dtype=np.uint8)
    for off in SCALE_FIELDS[wtype]:
        lo, hi = SCALE_RANGE[wtype]
        scale = (rng.uniform(lo, hi, (rows, nb)) * rng.choice([1.0, -1.0], (rows, nb))).astype("<f2")
        raw[:, :, off:off + 2] = scale.view(np.uint8).reshape(rows, nb, 2)
        if special:
            sel = rng.random((rows, nb)) < 0.2
            codes = rng.choice(SPECIAL_F16, (rows, nb)).astype("<u2").view(np.uint8).reshape(rows, nb, 2)
            raw[:, :, off:off + 2][sel] = codes[sel]
    return raw.reshape(rows, nb * bb)


def make_bias(rng, btype, rows):
    b = (rng.standard_normal(rows) * 0.1)
    return b.astype("<f4").view(np.uint8) if btype == O.GGUF_F32 else b.astype("<f2").view(np.uint8)
