"""Full-size forwards of the benchmark configurations against the committed golden digests.

cfg3 (1 x 128) and the 8 sampled sequences of cfg4 (256 x 160) carry the reference C program's
ALL STATES EXACT verdict; cfg5 (32 x 4096, stress model with saturating scores) is pinned by
the oracle alone (c/intref.c holds 512 RoPE rows).  Only the sampled sequences leave the GPU.
"""
import hashlib
import json
import os

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from eii import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = json.load(open(os.path.join(ROOT, "tests", "golden", "golden.json")))


def sha(t):
    return hashlib.sha256(np.ascontiguousarray(t.cpu().numpy(), dtype=np.int32).tobytes()).hexdigest()


def run_config(cfg, resid=True):
    from eii.engine import Engine
    kind = GOLDEN[cfg]["model"]
    ids = synth.token_ids(cfg)
    eng = Engine(synth.ensure_model(kind), rope_rows=max(512, ids.shape[1]))
    out = None
    try:
        # the embedding and residual states of the sampled sequences only (dump selection)
        sampled = sorted(int(b) for b in GOLDEN[cfg]["sequences"])
        out = eng.forward(ids, embed=True, resid=resid, logits=True, dump=sampled)
        torch.cuda.synchronize()
        bad = []
        for b, g in GOLDEN[cfg]["sequences"].items():
            b = int(b)
            j = sampled.index(b)
            print(f"{cfg} sequence {b}", flush=True)
            if sha(out["embed"][j]) != g["embed"]:
                bad.append((b, "embed"))
            if resid and sha(out["resid"][:, j]) != g["resid_out"]:
                bad.append((b, "resid_out"))
            if sha(out["logits"][b]) != g["logits"]:
                bad.append((b, "logits"))
            got_head = out["logits"][b, -1, :8].cpu().numpy().tolist()
            assert got_head == g["logits_last_row_head"] or (b, "logits") in bad
        return bad
    finally:
        del out
        eng.close()
        torch.cuda.empty_cache()


def test_cfg3_golden():
    assert run_config("cfg3") == []


def test_cfg4_golden_sampled():
    assert run_config("cfg4") == []


def test_cfg5_golden_sampled():
    # 131072 rows; the residual states of the 2 sampled sequences are 566 MB
    assert run_config("cfg5") == []
