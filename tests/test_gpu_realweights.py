"""Real-weight path end to end on the GPU: float checkpoint -> model.bin -> the reference's three
vector sets (t24, t128, t160) exported by the engine -> vectors.sha256, checked by eii_check and,
when built, by the reference's own C checker.  A synthetic bfloat16 checkpoint and token windows
stand in for the pinned assets, which are absent offline."""
import os
import subprocess

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CHECKER = os.path.join(ROOT, "exact-integer-inference_amd", "eii_check")
REF_BIN = os.path.join(ROOT, "oracle", "_ref", "intref")


@pytest.fixture(scope="module")
def sets(tmp_path_factory):
    from eii import realweights, synth
    d = tmp_path_factory.mktemp("real")
    synth.make_float_checkpoint(str(d / "model.safetensors"), seed=4)
    path = realweights.build_model_bin(str(d), str(d / "model.bin"), log=lambda s: None)
    windows = np.random.default_rng(4).integers(0, 49152, size=(101, realweights.SEQ_LEN), dtype=np.int64)
    out = d / "vectors"
    os.makedirs(out)
    assert realweights.export_sets(windows, path, str(out)) == 0
    return out


@pytest.mark.parametrize("name,T", [("t24", 24), ("t128", 128), ("t160", 160)])
def test_checker_accepts_exported_set(sets, name, T):
    print(name, flush=True)
    r = subprocess.run([CHECKER, str(sets / name)], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr
    assert r.stdout.strip().splitlines()[-1].startswith(f"ALL STATES EXACT ({T} tokens")


def test_hash_file(sets):
    from eii import export_vectors
    assert export_vectors.hash_root(str(sets), check=True) == 0
    names = sorted(l.split("  ", 1)[1] for l in open(sets / "vectors.sha256").read().split("\n") if l)
    assert names[0] == "model.bin" and "t160/exp_logits.i32" in names and len(names) == 16


@pytest.mark.skipif(not os.path.exists(REF_BIN), reason="oracle/_ref/intref not built")
@pytest.mark.parametrize("name", ["t24", "t128"])
def test_reference_checker_accepts_set(sets, name):
    r = subprocess.run([REF_BIN, str(sets / name)], capture_output=True, text=True, timeout=900)
    assert r.returncode == 0 and "ALL STATES EXACT" in r.stdout, r.stdout[-2000:]
