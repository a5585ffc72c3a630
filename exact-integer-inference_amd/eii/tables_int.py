"""Integer-only regeneration of the exp, SiLU and RoPE tables, with their digests.

The tables of the integer semantics are floor(v + 1/2) of real values fixed by closed forms
(python/intref.py:68-108), which the reference evaluates with 50-digit mpmath and which
eii/tables.py evaluates in float64 with an mpmath fallback near rounding boundaries.  This module
is a third, independent method using nothing but Python integers: every real value is carried
in fixed point with P = 512 fractional bits together with a bound on its error, and an entry is
accepted only when the whole error interval rounds to the same integer (otherwise
ArithmeticError; no entry of any table comes near that).

* exp(-d/128): e1 = exp(-1/128) by its Taylor series, E_d = E_{d-1} e1 (error grows by at most
  e1's error plus one unit per step).
* SiLU: x = q 2^-f_in, exp(-x) stepped from q = 0 by multiplication with exp(-+2^-f_in)
  (relative error grows by a few units per step), y = x / (1 + exp(-x)) by one integer division.
* RoPE: theta_j = 10^(-5j/32) = exp(-(5j/32) ln 10) with ln 10 = 3 ln 2 + ln(5/4) from atanh
  series, cos/sin of theta_j by Taylor series, then the angle p theta_j advances by rotation
  (complex multiplication by (cos theta_j, sin theta_j)), the error growing linearly in p.

The reference's own open item (docs/CONFORMANCE.md:19: "an independent cross-check of these
tables is open work") is this cross-check; tests/test_tables_int.py compares the three methods
entry by entry and pins the digests.

    python -m eii.tables_int [--model model.bin] [--rope-rows T]   # prints sha256 per table
"""
import argparse
import hashlib
import sys

import numpy as np

P = 512
ONE = 1 << P
DMAX = 1536
EXP_BITS = 30


def _rhu(X, s, err):
    """floor(x 2^s + 1/2) for x = X 2^-P known to within err units of 2^-P (s >= 0)."""
    t = (X << s) + (1 << (P - 1))
    e = err << s
    lo, hi = (t - e) >> P, (t + e) >> P
    if lo != hi:
        raise ArithmeticError("rounding undecided at this precision")
    return lo


def _exp_series(X):
    """exp(x) for x = X 2^-P, |x| <= 1: (value, error in units of 2^-P)."""
    s = term = ONE
    n = 0
    while term:
        n += 1
        term = term * X // (n << P)
        s += term
    return s, 2 * n + 2


def _atanh_inv(m):
    """atanh(1/m) for an integer m >= 2: (value, error)."""
    s = 0
    k = 0
    mm = m
    while True:
        term = ONE // (mm * (2 * k + 1))
        if not term:
            break
        s += term
        k += 1
        mm *= m * m
    return s, k + 3   # one unit per floor, and the tail after the last term (ratio 1/m^2) below two


def exp_table():
    """E[d] = floor(2^30 exp(-d/128) + 1/2), d = 0..1536 (python/intref.py:72-77)."""
    e1, err1 = _exp_series(-(ONE >> 7))
    out = np.empty(DMAX + 1, dtype=np.int64)
    E, err = ONE, 0
    for d in range(DMAX + 1):
        out[d] = _rhu(E, EXP_BITS, err)
        E = E * e1 >> P
        err = err + err1 + 1
    return out


def silu_table(f_in, f_out, out_bits):
    """SILU[q + 32768] = SAT(floor(2^f_out x / (1 + e^-x) + 1/2), out_bits), x = q 2^-f_in,
    q = -32768..32767 (python/intref.py:80-93)."""
    if f_in < 0 or f_in > 64 or f_out < 0 or f_out > 64:
        raise ValueError("formats outside 0..64")
    dn, err_dn = _exp_series(-(ONE >> f_in))   # exp(-2^-f_in)
    up, err_up = _exp_series(ONE >> f_in)      # exp(+2^-f_in)
    lo_sat, hi_sat = -(1 << (out_bits - 1)), (1 << (out_bits - 1)) - 1
    vals = np.empty(65536, dtype=np.int64)
    # relative error bound of exp(-x) after k steps: k (err + 2) units; y = x / (1 + exp(-x)) then
    # has an absolute error below |x| k (err + 2) + 1 units (d y / d e = -x / (1 + e)^2 and
    # e / (1 + e)^2 <= 1/4), plus one unit for the division
    step = max(err_dn, err_up) + 2

    def value(q, E, k):
        X = q << (P - f_in)
        Y = (X << P) // (ONE + E)
        err = (abs(q) >> f_in) * k * step + k * step + 2
        return min(max(_rhu(Y, f_out, err), lo_sat), hi_sat)

    E = ONE
    for q in range(0, 32768):
        vals[q + 32768] = value(q, E, q)
        E = E * dn >> P
    E = ONE
    for q in range(-1, -32769, -1):
        E = E * up >> P
        vals[q + 32768] = value(q, E, -q)
    return vals


def rope_tables(T):
    """C[p, j] = floor(2^30 cos(p theta_j) + 1/2), S likewise with sin, theta_j = 100000^(-2j/64),
    p = 0..T-1, j = 0..31 (python/intref.py:96-108)."""
    ln2, e2 = _atanh_inv(3)
    ln54, e54 = _atanh_inv(9)
    ln10 = 3 * 2 * ln2 + 2 * ln54          # ln 2 = 2 atanh(1/3), ln 5/4 = 2 atanh(1/9)
    err_ln10 = 6 * e2 + 2 * e54
    C = np.empty((T, 32), dtype=np.int64)
    S = np.empty((T, 32), dtype=np.int64)
    for j in range(32):
        a = 5 * j * ln10 // 32               # (5j/32) ln 10 <= 11.2
        err_a = 5 * j * err_ln10 // 32 + 2
        # exp(-a) = 1 / exp(a); exp(a) = exp(a / 16)^16 keeps the series argument below 1
        ea, err_ea = _exp_series(a >> 4)
        err_ea += ((err_a >> 4) + 2) * 3     # the argument's error, times exp(a / 16) < 3
        for _ in range(4):
            ea, err_ea = ea * ea >> P, 2 * err_ea * ((ea >> P) + 1) + 1
        theta = (ONE << P) // ea
        err_t = err_ea + 2                   # exp(a) >= 1, so dividing does not grow it
        # cos theta, sin theta (theta <= 1) by their Taylor series, with theta's error carried
        c = s_ = 0
        term = ONE
        n = 0
        while term:
            if n % 4 == 0:
                c += term
            elif n % 4 == 1:
                s_ += term
            elif n % 4 == 2:
                c -= term
            else:
                s_ -= term
            n += 1
            term = term * theta // (n << P)
        err_cs = 2 * n + 2 + err_t
        Cp, Sp, err = ONE, 0, 0
        for p in range(T):
            C[p, j] = _rhu(Cp, EXP_BITS, err)
            S[p, j] = _rhu(Sp, EXP_BITS, err)
            Cp, Sp = (Cp * c - Sp * s_) >> P, (Sp * c + Cp * s_) >> P
            err = err + 2 * err_cs + 4
    return C, S


def digest(a):
    return hashlib.sha256(np.ascontiguousarray(a, dtype="<i8").tobytes()).hexdigest()


def main(argv=None):
    ap = argparse.ArgumentParser(description="Regenerate the tables with integer arithmetic; print digests")
    ap.add_argument("--model", help="model.bin: the SiLU tables of its formats (default: none)")
    ap.add_argument("--rope-rows", type=int, default=512)
    a = ap.parse_args(argv)
    print(f"exp {digest(exp_table())}")
    C, S = rope_tables(a.rope_rows)
    print(f"rope{a.rope_rows}.cos {digest(C)}")
    print(f"rope{a.rope_rows}.sin {digest(S)}")
    if a.model:
        from . import modelbin as mb
        m = mb.read(a.model)
        seen = set()
        for l in range(mb.NL):
            key = (m.fmt("gate_proj", l)[1], m.fmt("silu_gate", l)[1], m.fmt("silu_gate", l)[0])
            if key not in seen:
                seen.add(key)
                print(f"silu f_in={key[0]} f_out={key[1]} bits={key[2]} {digest(silu_table(*key))}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
