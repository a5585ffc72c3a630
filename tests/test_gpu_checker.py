"""Conformance tooling on the GPU: eii.export_vectors writes vector directories, eii_check (the
`prog VECTORDIR [MODELDIR]` checker) accepts them and rejects a planted one-unit change, and
the reference's own C checker (when built into oracle/_ref/) accepts the same files."""
import os
import subprocess

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CHECKER = os.path.join(ROOT, "exact-integer-inference_amd", "eii_check")
REF_BIN = os.path.join(ROOT, "oracle", "_ref", "intref")


def run(args, timeout=600):
    print(" ".join(args), flush=True)
    return subprocess.run(args, capture_output=True, text=True, timeout=timeout)


@pytest.fixture(scope="module")
def vec(tmp_path_factory):
    from eii import export_vectors
    root = tmp_path_factory.mktemp("vectors")
    export_vectors.main([str(root / "t24"), "--config", "cfg1"])
    ids = np.random.default_rng(600).integers(0, 49152, size=600, dtype=np.int64)
    ids.astype("<i8").tofile(root / "ids600.i64")
    export_vectors.main([str(root / "t600"), "--ids", str(root / "ids600.i64"), "--window", "7"])
    return root


def test_checker_accepts_exported_vectors(vec):
    r = run([CHECKER, str(vec / "t24")])
    assert r.returncode == 0, r.stdout + r.stderr
    lines = r.stdout.strip().splitlines()
    assert lines[0].startswith("device: ")
    assert [l for l in lines if l.startswith("layer ")] == [f"layer {l:2d}: exact" for l in range(30)]
    assert "logits: exact" in lines and lines[-1].startswith("ALL STATES EXACT (24 tokens")


def test_checker_long_sequence_with_rope_rows(vec):
    # 600 tokens: the RoPE rows beyond model.bin's 512 come from the exported rope.i64
    assert os.path.getsize(vec / "t600" / "rope.i64") == 2 * 600 * 32 * 8
    r = run([CHECKER, str(vec / "t600")])
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().splitlines()[-1].startswith("ALL STATES EXACT (600 tokens")


def test_checker_reports_a_planted_difference(vec, tmp_path):
    d = tmp_path / "bad"
    d.mkdir()
    for name in ("ids.i64", "exp_embed.i32", "exp_logits.i32"):
        os.symlink(vec / "t24" / name, d / name)
    res = np.fromfile(vec / "t24" / "exp_resid_out.i32", dtype="<i4").reshape(30, 24, 576)
    res[7, 5, 100] += 1
    res.tofile(d / "exp_resid_out.i32")
    r = run([CHECKER, str(d), str(vec / "t24")])
    assert r.returncode == 1
    assert "  MISMATCH resid_out  1 of 13824, first at 2980" in r.stdout
    assert "layer  7: DIFFERS" in r.stdout and "layer  8" not in r.stdout
    assert r.stdout.strip().splitlines()[-1].startswith("FAIL (24 tokens")


def test_checker_usage_and_io_errors(tmp_path):
    assert run([CHECKER]).returncode == 2
    assert run([CHECKER, str(tmp_path)]).returncode == 2


def test_hash_and_manifest(vec):
    from eii import export_vectors
    assert export_vectors.main([str(vec), "--hash"]) == 0
    assert export_vectors.main([str(vec), "--hash", "--check"]) == 0
    import json
    man = json.load(open(vec / "t24" / "manifest.json"))
    assert man["tokens"] == 24 and man["window"] == 64
    assert man["files"]["exp_logits.i32"]["bytes"] == 24 * 49152 * 4


@pytest.mark.skipif(not os.path.exists(REF_BIN), reason="oracle/_ref/intref not built")
def test_reference_checker_accepts_gpu_vectors(vec):
    r = run([REF_BIN, str(vec / "t24")])
    assert r.returncode == 0 and "ALL STATES EXACT" in r.stdout, r.stdout[-2000:]


def test_conformance_record(vec, tmp_path):
    """python -m eii.conformance over the exported sets: hash check, the reference's C checker as
    the CPU check (when built, for the set it can read: T <= 512), eii_check, the planted +1."""
    from eii import conformance, export_vectors
    assert export_vectors.hash_root(str(vec)) == 0
    cpu = REF_BIN if os.path.exists(REF_BIN) else None
    status, path = conformance.record(str(vec), str(tmp_path / "runs"), sets=["t24"], cpu_checker=cpu,
                                      variants=(), timeout=240)
    text = open(path).read()
    print(text[-1500:])
    assert status == 0, text
    assert "negative test: detected" in text and "eii_check: pass" in text
    assert f"exact lines: {2 if cpu else 1} ({2 if cpu else 1} expected" in text
    status, path = conformance.record(str(vec), str(tmp_path / "runs2"), sets=["t24", "t600"], variants=(),
                                      timeout=240)
    assert status == 0, open(path).read()
