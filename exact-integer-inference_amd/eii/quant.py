"""Float weights to the integer formats of model.bin (python/intref.py:113-130).

These are the only floating-point steps between a checkpoint and the integer model, and their
results are part of the format: the same float64 operations in the same order (numpy's log2,
floor and round-half-even rint) give the same integers, so the steps are kept exactly as the
reference defines them.
"""
import math

import numpy as np

I64 = np.int64


def quant_rows(W):
    """W float [N, K] -> (q [N, K] int8 values held as float64, m int64 [N], n int64 [N]).

    Per row: scale s = max|w| / 127 (1 for an all-zero row), n = 13 - floor(log2 s) and
    m = rint(s 2^n) in [2^13, 2^14], so m 2^-n is s to 15 significant bits; q = clip(rint(w /
    (m 2^-n)), -127, 127) (python/intref.py:113-124).
    """
    W = np.asarray(W, dtype=np.float64)
    scale = np.abs(W).max(axis=1) / 127.0
    scale[scale == 0] = 1.0
    n = (13 - np.floor(np.log2(scale))).astype(I64)
    m = np.rint(scale * 2.0 ** n).astype(I64)
    if m.min() < 2 ** 13 or m.max() > 2 ** 14:
        raise AssertionError("row multiplier outside [2^13, 2^14]")
    step = m * 2.0 ** (-n.astype(np.float64))
    q = np.clip(np.rint(W / step[:, None]), -127, 127)
    return q, m, n


def quant_vec_int16(w):
    """Gain vector -> (q int64 in [-32768, 32767], f) with f = 14 - floor(log2 max|w|), q = rint(w 2^f)
    (python/intref.py:127-130)."""
    w = np.asarray(w, dtype=np.float64)
    f = 14 - int(math.floor(math.log2(np.abs(w).max())))
    return np.clip(np.rint(w * 2.0 ** f), -32768, 32767).astype(I64), f


def dequant(q, f):
    """q 2^-f as float64 (python/intref.py:311)."""
    return np.asarray(q, dtype=np.float64) * 2.0 ** (-f)
