"""The integer-only table generator (eii/tables_int.py) against the pinned digests and the two
floating-point methods: 50-digit mpmath (oracle/tables_ref.py, the arithmetic python/intref.py:68-108
uses) and the product's float64-with-fallback generator (eii/tables.py).

Three methods that share no code agreeing on every entry is the independent table regeneration
the reference lists as open work (docs/CONFORMANCE.md:19)."""
import hashlib
import json
import os

import numpy as np
import pytest

from eii import modelbin as mb
from eii import synth, tables, tables_int
from oracle import tables_ref

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = json.load(open(os.path.join(ROOT, "tests", "golden", "golden.json")))["tables"]


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a, dtype="<i8").tobytes()).hexdigest()


def test_exp_table():
    E = tables_int.exp_table()
    assert sha(E) == GOLDEN["exp"]
    assert np.array_equal(E, tables_ref.exp_table())
    assert int(E[0]) == 2 ** 30 and int(E[-1]) == int(tables_ref.exp_table()[-1])


def test_rope_4096_rows():
    C, S = tables_int.rope_tables(4096)
    assert (sha(C), sha(S)) == (GOLDEN["rope4096_cos"], GOLDEN["rope4096_sin"])
    assert (sha(C[:512]), sha(S[:512])) == (GOLDEN["rope512_cos"], GOLDEN["rope512_sin"])
    C0, S0 = tables_ref.rope_tables(4096, start=4090)
    assert np.array_equal(C0, C[4090:]) and np.array_equal(S0, S[4090:])


def test_silu_tables_of_the_models():
    """Every distinct (f_in, f_out, bits) of the synthetic models: the pinned digests and the tables
    stored in model.bin."""
    for kind in ("base", "stress"):
        m = mb.read(synth.ensure_model(kind))
        for l in range(mb.NL):
            (_, f_g), (b_s, f_s) = m.fmt("gate_proj", l), m.fmt("silu_gate", l)
            t = tables_int.silu_table(f_g, f_s, b_s)
            assert np.array_equal(t, np.asarray(m.layers[l]["silu"])), (kind, l)
            key = f"{f_g},{f_s},{b_s}"
            if key in GOLDEN["silu"]:
                assert sha(t) == GOLDEN["silu"][key], key


@pytest.mark.parametrize("f_in,f_out,bits", [(7, 7, 16), (12, 14, 16), (9, 20, 32), (13, 12, 16), (6, 30, 32)])
def test_silu_other_formats(f_in, f_out, bits):
    t = tables_int.silu_table(f_in, f_out, bits)
    assert np.array_equal(t, tables.silu_table(f_in, f_out, bits))
    # 50-digit mpmath on a sample: both ends, the neighbourhood of 0 and random entries
    idx = np.unique(np.concatenate([np.arange(0, 40), np.arange(32768 - 40, 32768 + 40), np.arange(65536 - 40, 65536),
                                    np.random.default_rng(f_in * 100 + f_out).integers(0, 65536, size=300)]))
    ref = tables_ref.silu_table(f_in, f_out, bits)
    assert np.array_equal(t[idx], ref[idx])


def test_cli_prints_digests(capsys):
    assert tables_int.main(["--rope-rows", "512"]) == 0
    out = capsys.readouterr().out.split("\n")
    assert out[0] == f"exp {GOLDEN['exp']}"
    assert out[1] == f"rope512.cos {GOLDEN['rope512_cos']}"
