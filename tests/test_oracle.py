"""Pins of the oracle (oracle/intref_np.py, oracle/tables_ref.py) and of the product's host tables.

Each check is chosen so that a plausible slip in the restatement fails it:
  * the reference's own C program (c/intref.c, compiled into oracle/_ref/) must accept the
    states the oracle exports for the 24-token case (every layer and the logits);
  * the committed golden digests (tests/golden/golden.json, written by make_golden.py, whose
    T <= 512 entries carry that C program's verdict) must be reproduced;
  * tiny cases are recomputed with Python integers straight from the definitions
    (python/intref.py:42-63,168-190,227-254), with math.isqrt and // as the exact routines;
  * planted mistakes in a copy of the oracle (tie rounding, GQA group, exp-table offset) must
    change the pinned states.
"""
import hashlib
import json
import math
import os
import subprocess
import tempfile

import numpy as np
import pytest

from eii import formats, synth, tables
from oracle import intref_np as O
from oracle import tables_ref

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = json.load(open(os.path.join(ROOT, "tests", "golden", "golden.json")))
REF_BIN = os.path.join(ROOT, "oracle", "_ref", "intref")


def sha(a, dt=np.int32):
    return hashlib.sha256(np.ascontiguousarray(a, dtype=dt).tobytes()).hexdigest()


@pytest.fixture(scope="module")
def cfg1_states(oracle):
    ids = synth.token_ids("cfg1")
    return ids, oracle.forward(ids)


# ------------------------------------------------------------------ golden vectors

def test_cfg1_golden(cfg1_states):
    _, (emb, res, lg) = cfg1_states
    g = GOLDEN["cfg1"]["sequences"]["0"]
    assert "ALL STATES EXACT" in g["reference_c"]
    assert sha(emb[0]) == g["embed"]
    assert sha(res[:, 0]) == g["resid_out"]
    assert sha(lg[0]) == g["logits"]


def test_cfg3_golden(oracle):
    ids = synth.token_ids("cfg3")
    emb, res, lg = oracle.forward(ids)
    g = GOLDEN["cfg3"]["sequences"]["0"]
    assert "ALL STATES EXACT" in g["reference_c"]
    assert (sha(emb[0]), sha(res[:, 0]), sha(lg[0])) == (g["embed"], g["resid_out"], g["logits"])


def test_cfg4_golden_two_sequences(oracle):
    ids = synth.token_ids("cfg4")
    for b in (0, 255):
        emb, res, lg = oracle.forward(ids[b:b + 1])
        g = GOLDEN["cfg4"]["sequences"][str(b)]
        assert "ALL STATES EXACT" in g["reference_c"]
        assert (sha(res[:, 0]), sha(lg[0])) == (g["resid_out"], g["logits"])


@pytest.mark.skipif(not os.path.exists(REF_BIN), reason="oracle/_ref/intref not built (make -C oracle ref)")
def test_reference_c_accepts_oracle_states(cfg1_states, model_path):
    ids, (emb, res, lg) = cfg1_states
    with tempfile.TemporaryDirectory() as d:
        ids[0].astype(np.int64).tofile(os.path.join(d, "ids.i64"))
        emb[0].astype(np.int32).tofile(os.path.join(d, "exp_embed.i32"))
        res[:, 0].astype(np.int32).tofile(os.path.join(d, "exp_resid_out.i32"))
        lg[0].astype(np.int32).tofile(os.path.join(d, "exp_logits.i32"))
        os.symlink(model_path, os.path.join(d, "model.bin"))
        r = subprocess.run([REF_BIN, d, d], capture_output=True, text=True, timeout=300)
        assert r.returncode == 0, r.stdout[-2000:]
        assert "ALL STATES EXACT" in r.stdout
        # the comparison is not vacuous: one changed logit is reported
        bad = lg[0].astype(np.int32).copy()
        bad[3, 17] += 1
        bad.tofile(os.path.join(d, "exp_logits.i32"))
        r = subprocess.run([REF_BIN, d, d], capture_output=True, text=True, timeout=300)
        assert r.returncode == 1 and "MISMATCH" in r.stdout


# ------------------------------------------------------------------ planted mistakes

def _planted(monkeypatch, oracle, what):
    if what == "rs_ties_down":
        def rs_bad(x, n):
            if np.isscalar(n) and int(n) <= 0:
                return x << (-int(n))
            n = np.asarray(n, dtype=np.int64)
            return (x + (np.int64(1) << (n - 1)) - 1) >> n      # ties toward -inf
        monkeypatch.setattr(O, "rs", rs_bad)
    elif what == "exp_offset":
        E = oracle.exp_tab.copy()
        monkeypatch.setattr(oracle, "exp_tab", np.concatenate([E[1:], [0]]))
    elif what == "gqa_group":
        real = oracle.attention

        def swapped(qr, kr, vv, *a, **k):
            return real(qr, kr[:, ::-1].copy(), vv[:, ::-1].copy(), *a, **k)
        monkeypatch.setattr(oracle, "attention", swapped)


@pytest.mark.parametrize("what", ["rs_ties_down", "exp_offset", "gqa_group"])
def test_planted_mistake_is_caught(monkeypatch, model_path, what):
    m = O.OracleModel(model_path)
    _planted(monkeypatch, m, what)
    ids = synth.token_ids("cfg1")
    emb, res, lg = m.forward(ids)
    g = GOLDEN["cfg1"]["sequences"]["0"]
    assert sha(res[:, 0]) != g["resid_out"] or sha(lg[0]) != g["logits"]


# ------------------------------------------------------------------ brute force on tiny cases

def rs_int(x, n):
    return x << (-n) if n <= 0 else (x + (1 << (n - 1))) >> n


def sat_int(x, bits):
    return min(max(x, -(1 << (bits - 1))), (1 << (bits - 1)) - 1)


def test_rs_sat_bruteforce():
    rng = np.random.default_rng(5)
    xs = rng.integers(-2 ** 40, 2 ** 40, size=400)
    for n in (-3, 0, 1, 2, 7, 16, 30):
        got = O.rs(xs.astype(np.int64), n)
        assert [int(v) for v in got] == [rs_int(int(x), n) for x in xs]
    nv = rng.integers(1, 40, size=400)
    got = O.rs(xs.astype(np.int64), nv)
    assert [int(v) for v in got] == [rs_int(int(x), int(n)) for x, n in zip(xs, nv)]
    for x in (-3, -2, -1, 1, 2, 3):                    # exact halves round toward +inf
        assert int(O.rs(np.int64(x), 1)) == math.floor(x / 2 + 0.5)
    vals = np.array([-2 ** 40, -32769, -32768, 0, 32767, 32768, 2 ** 40])
    assert [int(v) for v in O.sat(vals, 16)] == [sat_int(int(v), 16) for v in vals]


def test_rmsnorm_bruteforce(oracle):
    rng = np.random.default_rng(6)
    x = np.concatenate([rng.integers(-2 ** 31, 2 ** 31, size=(3, 576)),
                        rng.integers(-300, 300, size=(2, 576)),
                        np.zeros((1, 576), dtype=np.int64),
                        np.full((1, 576), -2 ** 31)]).astype(np.int64)
    gq = rng.integers(2 ** 13, 2 ** 14, size=576).astype(np.int64)
    fw, f_out, bits = 14, 11, 16
    got = oracle.rmsnorm(x, (gq, fw), f_out, bits)
    for t in range(x.shape[0]):
        S = sum(int(v) * int(v) for v in x[t])
        U = math.isqrt((1 << 80) // (S + O.EPS_S))
        z = [rs_int(int(v) * U, 16) for v in x[t]]
        want = [sat_int(rs_int(3 * zi * int(g), 21 + fw - f_out), bits) for zi, g in zip(z, gq)]
        assert [int(v) for v in got[t]] == want


def test_linear_bruteforce(oracle):
    rng = np.random.default_rng(7)
    a = rng.integers(-2 ** 15, 2 ** 15, size=(4, 64)).astype(np.int64)
    q = rng.integers(-127, 128, size=(8, 64)).astype(np.int64)
    m = rng.integers(2 ** 13, 2 ** 14 + 1, size=8).astype(np.int64)
    n = rng.integers(20, 26, size=8).astype(np.int64)
    out, acc = oracle.linear(a, 1 << 15, (q.astype(np.float64), m, n), 11, 10, 16)
    for t in range(4):
        for j in range(8):
            s = sum(int(a[t, k]) * int(q[j, k]) for k in range(64))
            assert int(acc[t, j]) == s
            assert int(out[t, j]) == sat_int(rs_int(s * int(m[j]), int(n[j]) + 11 - 10), 16)


def attention_int(qr, kr, vv, shift_s, f_v, f_c, bits_c, E):
    """python/intref.py:227-254 with Python integers, one sequence."""
    T = qr.shape[0]
    out = np.zeros((T, 9, 64), dtype=np.int64)
    for hh in range(9):
        g = hh // 3
        for i in range(T):
            s = [sat_int(rs_int(sum(int(qr[i, hh, d]) * int(kr[j, g, d]) for d in range(64)), shift_s), 16)
                 for j in range(i + 1)]
            mx = max(s)
            e = [int(E[mx - sj]) if mx - sj <= O.DMAX else 0 for sj in s]
            Z = sum(e)
            P = [(ej * 65536 + Z // 2) // Z for ej in e]
            for d in range(64):
                acc = sum(P[j] * int(vv[j, g, d]) for j in range(i + 1))
                out[i, hh, d] = sat_int(rs_int(acc, 16 + f_v - f_c), bits_c)
    return out


@pytest.mark.parametrize("scale", [2 ** 9, 2 ** 15])
def test_attention_bruteforce(oracle, scale):
    rng = np.random.default_rng(8 + scale)
    T = 6
    lim = min(scale, 2 ** 15)
    qr = rng.integers(-lim, lim, size=(T, 9, 64)).astype(np.int64)
    kr = rng.integers(-lim, lim, size=(T, 3, 64)).astype(np.int64)
    vv = rng.integers(-2 ** 15, 2 ** 15, size=(T, 3, 64)).astype(np.int64)
    shift_s, f_v, f_c, bits_c = 16, 11, 11, 16
    got = oracle.attention(qr, kr, vv, shift_s, f_v, f_c, bits_c, 16, 16, 16)
    want = attention_int(qr, kr, vv, shift_s, f_v, f_c, bits_c, oracle.exp_tab)
    assert np.array_equal(got.reshape(T, 9, 64), want)


def test_attention_probability_invariants(oracle):
    """Sum_j P_j lies in [65536 - T/2, 65536 + T/2]; one surviving key gets exactly 65536."""
    E = oracle.exp_tab
    rng = np.random.default_rng(9)
    for T in (1, 2, 7, 100, 1000):
        d = rng.integers(0, 1700, size=T)
        d[0] = 0
        e = np.where(d <= O.DMAX, E[np.clip(d, 0, O.DMAX)], 0)
        Z = int(e.sum())
        P = (e * 65536 + Z // 2) // Z
        assert 65536 - T / 2 <= int(P.sum()) <= 65536 + T / 2
        if (e > 0).sum() == 1:
            assert int(P.max()) == 65536


# ------------------------------------------------------------------ tables and formats

def test_tables_against_golden():
    g = GOLDEN["tables"]
    assert sha(tables_ref.exp_table(), np.int64) == g["exp"]
    assert sha(tables.exp_table(), np.int64) == g["exp"]
    for key, digest in g["silu"].items():
        f_g, f_s, bits = (int(v) for v in key.split(","))
        assert sha(tables.silu_table(f_g, f_s, bits), np.int64) == digest, key
    C, S = tables.rope_tables(4096)
    assert (sha(C, np.int64), sha(S, np.int64)) == (g["rope4096_cos"], g["rope4096_sin"])
    assert (sha(C[:512], np.int64), sha(S[:512], np.int64)) == (g["rope512_cos"], g["rope512_sin"])


def test_tables_ref_matches_product_tables():
    """The mpmath restatement and the product's float64-with-fallback generator agree."""
    assert np.array_equal(tables_ref.silu_table(11, 12, 16), tables.silu_table(11, 12, 16))
    assert np.array_equal(tables_ref.silu_table(8, 24, 32), tables.silu_table(8, 24, 32))
    C0, S0 = tables_ref.rope_tables(4096, start=4088)
    C, S = tables.rope_tables(4096)
    assert np.array_equal(C0, C[4088:]) and np.array_equal(S0, S[4088:])


def test_table_closed_forms():
    E = tables_ref.exp_table()
    assert int(E[0]) == 2 ** 30 and len(E) == O.DMAX + 1
    assert int(E[128]) == math.floor(2 ** 30 / math.e + 0.5)
    assert np.all(np.diff(E) <= 0)
    s = tables.silu_table(10, 10, 16)
    assert int(s[32768]) == 0                                # silu(0) = 0
    assert int(s[32768 + 1024]) == round(1024 / (1 + math.exp(-1)))   # silu(1) in Q10
    C, S = tables.rope_tables(2)
    assert np.all(C[0] == 2 ** 30) and np.all(S[0] == 0)
    assert int(C[1, 0]) == math.floor(math.cos(1.0) * 2 ** 30 + 0.5)


def test_formats_match_proposal():
    fm, f_y = formats.load_fm()
    assert f_y == 8
    cell = lambda l, site: (int(fm[l][2 * site]), int(fm[l][2 * site + 1]))
    assert cell(0, 6) == (32, 30) and cell(4, 6) == (32, 27)        # attn_ctx flagged at 0 and 4
    assert cell(11, 10) == (32, 24) and cell(28, 10) == (32, 24)    # silu_gate flagged at 11 and 28
    assert cell(29, 9) == (16, 7) and cell(0, 0) == (16, 13)
    flagged = {s: sum(fm[l][2 * s] == 32 for l in range(30)) for s in range(12)}
    assert flagged[11] == 26 and flagged[6] == 2 and flagged[10] == 2
    assert all(flagged[s] == 0 for s in (0, 1, 2, 3, 4, 5, 7, 8, 9))
