"""The C restatement (oracle/intref_c.c) against the golden digests and the numpy oracle.

Two independent restatements of python/intref.py agreeing bit for bit pins the cases the
reference's own C program cannot check (sequences longer than its 512 RoPE rows).
"""
import hashlib
import json
import os
import subprocess

import numpy as np
import pytest

from eii import synth
from eii.tables import rope_tables

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "oracle", "_build", "intref_c")
GOLDEN = json.load(open(os.path.join(ROOT, "tests", "golden", "golden.json")))


@pytest.fixture(scope="module", autouse=True)
def built():
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)


def sha(path):
    return hashlib.sha256(open(path, "rb").read()).hexdigest()


def run_c(d, ids, model_path):
    ids.astype("<i8").tofile(os.path.join(d, "ids.i64"))
    os.symlink(model_path, os.path.join(d, "model.bin"))
    if ids.size > 512:
        C, S = rope_tables(ids.size)
        np.concatenate([C.reshape(-1), S.reshape(-1)]).astype("<i8").tofile(os.path.join(d, "rope.i64"))
    r = subprocess.run([BIN, str(d)], capture_output=True, text=True, timeout=3600)
    assert r.returncode == 0 and r.stdout.startswith("WROTE STATES"), r.stdout + r.stderr
    return r


@pytest.mark.parametrize("cfg,seq", [("cfg1", 0), ("cfg3", 0), ("cfg4", 37), ("cfg4", 222)])
def test_golden(tmp_path, cfg, seq):
    g = GOLDEN[cfg]["sequences"][str(seq)]
    run_c(tmp_path, synth.token_ids(cfg)[seq], synth.ensure_model(GOLDEN[cfg]["model"]))
    assert sha(tmp_path / "exp_embed.i32") == g["embed"]
    assert sha(tmp_path / "exp_resid_out.i32") == g["resid_out"]
    assert sha(tmp_path / "exp_logits.i32") == g["logits"]


def test_check_mode_grammar(tmp_path):
    run_c(tmp_path, synth.token_ids("cfg1")[0], synth.ensure_model("base"))
    r = subprocess.run([BIN, str(tmp_path)], capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.strip().splitlines()[-1].startswith("ALL STATES EXACT (24 tokens")
    lg = np.fromfile(tmp_path / "exp_logits.i32", dtype="<i4")
    lg[1000] -= 1
    lg.tofile(tmp_path / "exp_logits.i32")
    r = subprocess.run([BIN, str(tmp_path)], capture_output=True, text=True)
    assert r.returncode == 1
    assert "  MISMATCH logits       1 of 1179648, first at 1000" in r.stdout and "logits: DIFFERS" in r.stdout


def test_agrees_with_numpy_oracle_on_stress_model(tmp_path, stress_model_path):
    """Saturating scores and many keys beyond the exp table: both restatements, state by state."""
    from oracle.intref_np import OracleModel
    ids = np.random.default_rng(77).integers(0, 49152, size=40, dtype=np.int64)
    run_c(tmp_path, ids, stress_model_path)
    emb, res, lg = OracleModel(stress_model_path).forward(ids[None, :])
    assert np.array_equal(np.fromfile(tmp_path / "exp_embed.i32", dtype="<i4").reshape(40, 576), emb[0])
    assert np.array_equal(np.fromfile(tmp_path / "exp_resid_out.i32", dtype="<i4").reshape(30, 40, 576), res[:, 0])
    assert np.array_equal(np.fromfile(tmp_path / "exp_logits.i32", dtype="<i4").reshape(40, 49152), lg[0])


@pytest.mark.slow
@pytest.mark.skipif(not os.environ.get("EII_SLOW"), reason="minutes of CPU per sequence; set EII_SLOW=1")
@pytest.mark.parametrize("seq", [0, 31])
def test_cfg5_golden(tmp_path, seq):
    g = GOLDEN["cfg5"]["sequences"][str(seq)]
    run_c(tmp_path, synth.token_ids("cfg5")[seq], synth.ensure_model("stress"))
    assert sha(tmp_path / "exp_resid_out.i32") == g["resid_out"]
    assert sha(tmp_path / "exp_logits.i32") == g["logits"]
