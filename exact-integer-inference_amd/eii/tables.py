"""Exact lookup tables of the integer semantics: exp, SiLU and RoPE.

Each entry is floor(v + 1/2) of a real value v fixed by a closed form
(python/intref.py:68-108): the rounding is of the exact real number, so any method
that decides the rounding correctly gives the same integers.  Here float64 decides
it wherever the float64 value sits clearly away from a rounding boundary, and
50-digit mpmath (the arithmetic python/intref.py:28 uses) decides the rest.
The float64 error bound used for "clearly away" is stated per table below.
"""
import math

import numpy as np
import mpmath as mp

from .modelbin import DMAX

EXP_BITS = 30
_MP_DPS = 50


def _rhu_mp(v):
    return int(mp.floor(v + mp.mpf(1) / 2))


def _round_checked(v, err, exact_fn):
    """Round float64 values v half up where |frac - 1/2| > err; call exact_fn(i) elsewhere."""
    v = np.asarray(v, dtype=np.float64)
    r = np.floor(v + 0.5)
    frac = v - np.floor(v)
    risky = np.abs(frac - 0.5) <= err
    out = r.astype(np.int64)
    if risky.any():
        with mp.workdps(_MP_DPS):
            for i in np.flatnonzero(risky.ravel()):
                out.flat[i] = exact_fn(int(i))
    return out


_exp = None


def exp_table():
    """E[d] = floor(2^30 * exp(-d/128) + 1/2), d = 0..1536 (python/intref.py:72-77)."""
    global _exp
    if _exp is None:
        with mp.workdps(_MP_DPS):
            _exp = np.array([_rhu_mp(mp.mpf(2) ** EXP_BITS * mp.exp(-mp.mpf(d) / 128))
                             for d in range(DMAX + 1)], dtype=np.int64)
    return _exp


_silu = {}


def silu_table(f_in, f_out, out_bits):
    """SILU[q + 32768] = SAT(floor(2^f_out * x/(1+e^-x) + 1/2), out_bits), x = q * 2^-f_in,
    q = -32768..32767 (python/intref.py:80-93).

    float64 evaluates x/(1+e^-x)*2^f_out with relative error below 2^-48, so entries whose
    fractional part lies farther than |v| * 2^-44 + 2^-30 from one half round correctly.
    """
    key = (int(f_in), int(f_out), int(out_bits))
    if key not in _silu:
        q = np.arange(-32768, 32768, dtype=np.float64)
        x = q * 2.0 ** (-f_in)
        with np.errstate(over="ignore"):
            v = x / (1.0 + np.exp(-x)) * 2.0 ** f_out
        err = np.abs(v) * 2.0 ** -44 + 2.0 ** -30

        def exact(i):
            xm = mp.mpf(i - 32768) * mp.mpf(2) ** (-f_in)
            return _rhu_mp(xm / (1 + mp.exp(-xm)) * mp.mpf(2) ** f_out)

        vals = _round_checked(v, err, exact)
        lo, hi = -(1 << (out_bits - 1)), (1 << (out_bits - 1)) - 1
        _silu[key] = np.clip(vals, lo, hi)
    return _silu[key]


_rope = {}


def rope_tables(T, theta=100000, head_dim=64):
    """C[p, j] = floor(2^30 cos(p * theta^(-2j/64)) + 1/2) and S likewise with sin,
    p = 0..T-1, j = 0..31 (python/intref.py:96-108).

    The float64 angle p * inv_j carries an absolute error below p * 2^-51, so the scaled
    cos/sin carry an error below 2^30 * (p * 2^-51 + 2^-52); entries farther than twice that
    from one half round correctly.
    """
    key = (int(T), int(theta), int(head_dim))
    if key not in _rope:
        half = head_dim // 2
        with mp.workdps(_MP_DPS):
            inv_mp = [mp.mpf(theta) ** (-mp.mpf(2 * j) / head_dim) for j in range(half)]
        inv = np.array([float(a) for a in inv_mp])
        p = np.arange(T, dtype=np.float64)[:, None]
        ang = p * inv[None, :]
        err = 2.0 * (2.0 ** 30) * (p * 2.0 ** -51 + 2.0 ** -52) * np.ones_like(ang)

        def exact_c(i):
            pp, j = divmod(i, half)
            return _rhu_mp(mp.cos(pp * inv_mp[j]) * 2 ** 30)

        def exact_s(i):
            pp, j = divmod(i, half)
            return _rhu_mp(mp.sin(pp * inv_mp[j]) * 2 ** 30)

        C = _round_checked(np.cos(ang) * 2.0 ** 30, err, exact_c)
        S = _round_checked(np.sin(ang) * 2.0 ** 30, err, exact_s)
        _rope[key] = (C, S)
    return _rope[key]
