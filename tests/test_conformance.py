"""The conformance record tool (eii/conformance.py, the steps of tools/record_conformance.sh:17-84)
on the CPU: its negative test, hash check, exact-line count and failure handling, driven with a
stand-in checker that compares the expected states with known-true copies and speaks the
checker's stdout grammar and exit codes.  The same tool over eii_check runs in
tests/test_gpu_checker.py."""
import os
import stat
import sys

import numpy as np
import pytest

from eii import conformance
from eii.export_vectors import hash_root

CHECKER_TEMPLATE = """#!{python}
import os, sys
import numpy as np
vec = sys.argv[1]
model = sys.argv[2] if len(sys.argv) > 2 else vec
mode = {mode!r}
if mode == "device-error":
    print("device: none", flush=True)
    sys.exit(3)
print("device: stand-in")
T = os.path.getsize(os.path.join(vec, "ids.i64")) // 8
got = np.fromfile(os.path.join(model, "truth_%d.i32" % T), dtype="<i4")
exp = np.fromfile(os.path.join(vec, "exp_resid_out.i32"), dtype="<i4")
bad = np.flatnonzero(got != exp)
if mode == "lenient" or bad.size == 0:
    print("layer  0: exact")
    print("ALL STATES EXACT (%d tokens, 0.0 s)" % T)
    sys.exit(0)
i = int(bad[0])
print("  MISMATCH resid_out  %d of %d, first at %d (got %d expected %d)" % (bad.size, exp.size, i, got[i], exp[i]))
print("layer  0: DIFFERS")
print("FAIL")
sys.exit(1)
"""


def make_checker(tmp_path, mode="strict"):
    p = tmp_path / f"checker_{mode}"
    p.write_text(CHECKER_TEMPLATE.format(python=sys.executable, mode=mode))
    p.chmod(p.stat().st_mode | stat.S_IXUSR)
    return str(p)


@pytest.fixture
def vecroot(tmp_path):
    root = tmp_path / "vectors"
    root.mkdir()
    (root / "model.bin").write_bytes(b"\0" * 64)
    rng = np.random.default_rng(3)
    for name, T in (("t24", 24), ("t128", 128)):
        d = root / name
        d.mkdir()
        np.arange(T, dtype="<i8").tofile(d / "ids.i64")
        res = rng.integers(-2 ** 31, 2 ** 31, size=3 * T, dtype=np.int64).astype("<i4")
        res.tofile(d / "exp_resid_out.i32")
        res.tofile(root / f"truth_{T}.i32")
        (d / "manifest.json").write_text('{"tokens": %d}' % T)
    hash_root(str(root))
    return root


def test_plant_one_unit(tmp_path):
    p = tmp_path / "a.i32"
    a = np.arange(-5, 5, dtype="<i4")
    a.tofile(p)
    assert conformance.plant_one_unit(str(p)) == 20
    b = np.fromfile(p, dtype="<i4")
    assert b[5] == a[5] + 1 and np.array_equal(np.delete(b, 5), np.delete(a, 5))
    # an odd size: the aligned word at or below the middle byte
    q = tmp_path / "b.bin"
    q.write_bytes(bytes(range(42)))
    assert conformance.plant_one_unit(str(q)) == 20
    assert q.read_bytes()[20:24] == (int.from_bytes(bytes(range(20, 24)), "little") + 1).to_bytes(4, "little")
    # a carry across bytes and a sign change
    r = tmp_path / "c.i32"
    np.array([0, 0, -1, 0], dtype="<i4").tofile(r)
    conformance.plant_one_unit(str(r))
    assert np.fromfile(r, dtype="<i4").tolist() == [0, 0, 0, 0]


def test_record_ok(vecroot, tmp_path):
    chk = make_checker(tmp_path)
    status, path = conformance.record(str(vecroot), str(tmp_path / "runs"), cpu_checker=chk, variants=(),
                                      checker=chk)
    text = open(path).read()
    assert status == 0, text
    assert "vectors match vectors.sha256" in text
    assert "exact lines: 4 (4 expected" in text
    assert "negative test: detected" in text and "  MISMATCH resid_out  1 of 72, first at 36" in text
    assert "sets: t24 t128" in text and "gpu: stand-in" in text
    assert text.rstrip().splitlines()[-2] == "RECORD OK"
    # the planted copy did not touch the original set
    assert np.array_equal(np.fromfile(vecroot / "t24" / "exp_resid_out.i32", dtype="<i4"),
                          np.fromfile(vecroot / "truth_24.i32", dtype="<i4"))


def test_record_hash_mismatch(vecroot, tmp_path):
    chk = make_checker(tmp_path)
    (vecroot / "t128" / "manifest.json").write_text("{}")
    status, path = conformance.record(str(vecroot), str(tmp_path / "runs"), variants=(), checker=chk)
    text = open(path).read()
    assert status == 1 and "VECTOR HASH MISMATCH" in text and "RECORD HAS FAILURES" in text


def test_record_checker_that_cannot_fail(vecroot, tmp_path):
    chk = make_checker(tmp_path, "lenient")
    status, path = conformance.record(str(vecroot), str(tmp_path / "runs"), variants=(), checker=chk)
    text = open(path).read()
    assert status == 1 and "negative test: NOT DETECTED" in text


def test_record_wrong_states(vecroot, tmp_path):
    chk = make_checker(tmp_path)
    np.fromfile(vecroot / "truth_24.i32", dtype="<i4")[::-1].tofile(vecroot / "truth_24.i32")
    status, path = conformance.record(str(vecroot), str(tmp_path / "runs"), variants=(), checker=chk)
    text = open(path).read()
    assert status == 1 and "eii_check: FAIL" in text and "exact lines: 1 (2 expected" in text


def test_record_stops_device_steps_after_a_device_error(vecroot, tmp_path):
    chk = make_checker(tmp_path, "device-error")
    status, path = conformance.record(str(vecroot), str(tmp_path / "runs"), variants=("-O1",), checker=chk)
    text = open(path).read()
    assert status == 1
    assert text.count("$ " + chk) == 1   # the second set, the negative test and the variant never ran
    assert "negative test: not run" in text and "variant [-O1]: not run" in text


def test_cli_no_sets(tmp_path):
    assert conformance.main([str(tmp_path), "--record-dir", str(tmp_path / "runs"), "--no-variants"]) == 1
    (rec,) = os.listdir(tmp_path / "runs")
    assert rec.startswith("run-") and rec.endswith(".txt")
