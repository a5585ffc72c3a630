"""The kernels' integer helpers (csrc/eii_int.h, host build) against exact Python integers."""
import ctypes as C
import math

import numpy as np
import pytest

from eii import lib as L

EPS_S = 6184753


@pytest.fixture(scope="module")
def hc():
    return L.load_hostcheck()


def rs_ref(x, n):                                    # python/intref.py:42-50, scalar n
    if n <= 0:
        return x << (-n)
    return (x + (1 << (n - 1))) >> n


def test_rs_sat(hc):
    rng = np.random.default_rng(0)
    for _ in range(20000):
        n = int(rng.integers(-20, 63))
        lim = 2 ** 62 >> max(0, -n)
        x = int(rng.integers(-lim, lim))
        assert hc.eii_host_rs(x, n) == rs_ref(x, n)
    for x in (-7, -6, -5, -4, -3, -2, -1, 0, 1, 2, 3, 5, 6, 7):      # ties go toward +inf
        assert hc.eii_host_rs(x, 1) == math.floor((x + 1) / 2)
    for bits in (8, 16, 32):
        lo, hi = -(1 << (bits - 1)), (1 << (bits - 1)) - 1
        for x in (lo - 1, lo, lo + 1, -1, 0, 1, hi - 1, hi, hi + 1, 2 ** 62, -2 ** 62):
            assert hc.eii_host_sat(x, bits) == min(max(x, lo), hi)
    assert hc.eii_host_sat(2 ** 62, 64) == 2 ** 62


def norm_U_ref(x):
    """python/intref.py:170-177 on one row of Python ints."""
    hi = [v >> 16 for v in x]
    lo = [v & 0xFFFF for v in x]
    A = sum(h * h for h in hi); B = sum(h * l for h, l in zip(hi, lo)); Cc = sum(l * l for l in lo)
    S = (A << 32) + (B << 17) + Cc
    assert S == sum(v * v for v in x)                # the three partial sums are exact
    return A, B, Cc, math.isqrt((1 << 80) // (S + EPS_S))


def test_norm_U(hc):
    rng = np.random.default_rng(1)
    rows = [[0] * 576, [-2 ** 31] * 576, [2 ** 31 - 1] * 576, [1] + [0] * 575, [-1] * 576]
    for scale in (1, 3, 2 ** 8, 2 ** 15, 2 ** 20, 2 ** 31):
        for _ in range(40):
            rows.append([int(v) for v in rng.integers(-scale, scale, size=576)])
    # rows whose S + EPS sits next to a boundary of the isqrt or the division
    for u in (11, 12, 1000, 2 ** 20 + 7, 2 ** 28):
        T = (1 << 80) // (u * u)
        for d in (-1, 0, 1):
            S = T + d - EPS_S
            if S >= 0:
                a = math.isqrt(S)
                rows.append([a, int(math.isqrt(S - a * a))] + [0] * 574)
    for x in rows:
        A, B, Cc, U = norm_U_ref(x)
        assert hc.eii_host_norm_U(A, B, Cc) == U, x[:4]


def test_norm_U_many_sums(hc):
    # 20000 row sums S over all magnitudes (Tt from EPS up to 2^73): the float64 estimate's floor,
    # taken directly when its fractional part is far from 0 and 1, and the exact tests otherwise
    rng = np.random.default_rng(5)
    for _ in range(20000):
        S = int(rng.integers(0, 2 ** 62)) >> int(rng.integers(0, 62))
        S = S * (1 << int(rng.integers(0, 12)))
        A, rem = divmod(S, 1 << 32)
        want = math.isqrt((1 << 80) // (S + EPS_S))
        assert hc.eii_host_norm_U(A, 0, rem) == want, S


def test_norm_U_boundaries_direct(hc):
    # Tt = S + EPS exactly at u^2 * Tt == 2^80 and one either side, with S given by A,B,C = (0,0,S)
    for u in (11, 64, 4096, 2 ** 20, 2 ** 25):
        if (1 << 80) % (u * u) == 0:
            Tt = (1 << 80) // (u * u)
            for d in (-1, 0, 1):
                S = Tt + d - EPS_S
                A, rem = divmod(S, 1 << 32)
                want = math.isqrt((1 << 80) // (S + EPS_S))
                assert hc.eii_host_norm_U(A, 0, rem) == want


def test_attn_prob(hc):
    rng = np.random.default_rng(2)
    cases = [(0, 2 ** 30), (2 ** 30, 2 ** 30), (2 ** 30, 2 ** 30 + 6596), (6596, 2 ** 30 + 6596),
             (2 ** 30, 2 ** 30 * 4096), (1, 2 ** 42 - 1)]
    for _ in range(20000):
        Z = int(rng.integers(2 ** 30, 2 ** 43))
        e = int(rng.integers(0, min(Z, 2 ** 30) + 1))
        cases.append((e, Z))
    for _ in range(2000):                         # quotients exactly at and next to integers
        Z = int(rng.integers(2 ** 30, 2 ** 40))
        P = int(rng.integers(0, 65537))
        num = P * Z
        e = (num - Z // 2) // 65536
        for de in (-1, 0, 1):
            if 0 <= e + de <= Z:
                cases.append((e + de, Z))
    for e, Z in cases:
        assert hc.eii_host_attn_prob(e, Z) == (e * 65536 + Z // 2) // Z, (e, Z)


@pytest.mark.parametrize("W", [2, 4])
def test_limb_dot(hc, W):
    rng = np.random.default_rng(W)
    bits = 8 * W
    for K in (1, 64, 576, 1536):
        a = rng.integers(-2 ** (bits - 1), 2 ** (bits - 1), size=K, dtype=np.int64).astype(np.int32)
        a[:2] = [-2 ** (bits - 1), 2 ** (bits - 1) - 1] if K >= 2 else a[:2]
        w = rng.integers(-128, 128, size=K, dtype=np.int64).astype(np.int8)
        want = int(np.dot(a.astype(np.int64), w.astype(np.int64)))
        got = hc.eii_host_limb_dot(a.ctypes.data_as(C.c_void_p), w.ctypes.data_as(C.c_void_p), K, W)
        assert got == want
