"""ORACLE (test infrastructure only): the reference's table closed forms in 50-digit mpmath.

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg use this module, as a
checker.  It restates python/intref.py:68-108 entry by entry with mpmath at 50 digits
(python/intref.py:28), the same arithmetic and version (mpmath 1.3.0, requirements.txt:8)
the reference uses, so its outputs are the reference's tables.

Pinned by: closed-form special cases (E[0] = 2^30, S[0, :] = 0, C[0, :] = 2^30, SILU(0) = 0,
SILU(x) -> x for large x, SILU(x) -> 0 for very negative x), an independent float64
evaluation that agrees within rounding everywhere (tests/test_tables.py), and the
committed sha256 digests in tests/golden/tables.json.
"""
import numpy as np
import mpmath as mp

DMAX = 12 * 128
EXP_BITS = 30


def _rhu(v):                                        # python/intref.py:68-69
    return int(mp.floor(v + mp.mpf(1) / 2))


def exp_table():                                    # python/intref.py:72-77
    with mp.workdps(50):
        return np.array([_rhu(mp.mpf(2) ** EXP_BITS * mp.exp(-mp.mpf(d) / 128))
                         for d in range(DMAX + 1)], dtype=np.int64)


def silu_table(f_in, f_out, out_bits):              # python/intref.py:80-93
    vals = np.empty(65536, dtype=np.int64)
    with mp.workdps(50):
        sc_in = mp.mpf(2) ** (-f_in)
        sc_out = mp.mpf(2) ** f_out
        for i in range(65536):
            x = (i - 32768) * sc_in
            y = x / (1 + mp.exp(-x))
            vals[i] = _rhu(y * sc_out)
    lo, hi = -(1 << (out_bits - 1)), (1 << (out_bits - 1)) - 1
    return np.clip(vals, lo, hi)


def rope_tables(T, theta=100000, head_dim=64, start=0):   # python/intref.py:96-108
    """Rows p = start..T-1 of the Q30 cos/sin tables."""
    half = head_dim // 2
    C = np.empty((T - start, half), dtype=np.int64)
    S = np.empty((T - start, half), dtype=np.int64)
    with mp.workdps(50):
        inv = [mp.mpf(theta) ** (-mp.mpf(2 * j) / head_dim) for j in range(half)]
        for p in range(start, T):
            for j in range(half):
                a = p * inv[j]
                C[p - start, j] = _rhu(mp.cos(a) * 2 ** 30)
                S[p - start, j] = _rhu(mp.sin(a) * 2 ** 30)
    return C, S
