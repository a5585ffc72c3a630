"""Export conformance vectors computed on the GPU, and hash them.

    python -m eii.export_vectors OUTDIR --config cfg1 [--seq 0] [--model model.bin]
    python -m eii.export_vectors OUTDIR --ids ids.i64 [--window W] [--model model.bin]
    python -m eii.export_vectors --hash ROOT [--check]

The first two forms follow python/export_vectors.py:15-66: OUTDIR receives ids.i64 and the
expected states exp_embed.i32 [T, 576], exp_resid_out.i32 [30, T, 576], exp_logits.i32
[T, 49152] (little-endian), computed by the engine, plus manifest.json {"window", "tokens",
"files": {name: {bytes, sha256}}} and, next to OUTDIR's files, model.bin (a symbolic link to
the model used) and for T > 512 rope.i64 (cos then sin, int64 [T, 32]) so that a checker can
load the rows model.bin does not hold.  The checkers (eii_check, c/intref.c) take
`OUTDIR [MODELDIR]`.

--hash writes ROOT/vectors.sha256 in sha256sum format over ROOT/model.bin,
ROOT/*/ids.i64, ROOT/*/exp_*.i32 and ROOT/*/manifest.json, the file set of
tools/hash_vectors.sh:10-13; --check verifies it.
"""
import argparse
import glob
import hashlib
import json
import os
import sys

import numpy as np

from . import modelbin as mb
from . import synth
from .tables import rope_tables


def sha256_file(path):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 22), b""):
            h.update(chunk)
    return h.hexdigest()


def export(outdir, ids, window, model_path):
    from .engine import Engine
    ids = np.ascontiguousarray(ids, dtype=np.int64).reshape(-1)
    T = ids.size
    os.makedirs(outdir, exist_ok=True)
    eng = Engine(model_path, rope_rows=max(mb.ROPE_POS, T))
    try:
        out = eng.forward(ids[None, :], embed=True, resid=True, logits=True)
        files = {
            "ids.i64": ids,
            "exp_embed.i32": out["embed"][0].cpu().numpy(),
            "exp_resid_out.i32": out["resid"][:, 0].cpu().numpy(),
            "exp_logits.i32": out["logits"][0].cpu().numpy(),
        }
    finally:
        eng.close()
    for name, arr in files.items():
        arr.astype("<i8" if name.endswith(".i64") else "<i4").tofile(os.path.join(outdir, name))
    link = os.path.join(outdir, "model.bin")
    if os.path.lexists(link):
        os.remove(link)
    os.symlink(os.path.abspath(model_path), link)
    if T > mb.ROPE_POS:
        C, S = rope_tables(T)
        np.concatenate([C.reshape(-1), S.reshape(-1)]).astype("<i8").tofile(os.path.join(outdir, "rope.i64"))
    man = {"window": window, "tokens": T, "files": {}}
    for name in sorted(files):
        p = os.path.join(outdir, name)
        man["files"][name] = {"bytes": os.path.getsize(p), "sha256": sha256_file(p)}
    with open(os.path.join(outdir, "manifest.json"), "w") as f:
        json.dump(man, f, indent=1)
    return man


def hash_root(root, check=False):
    out = os.path.join(root, "vectors.sha256")
    names = sorted(p for p in ([os.path.join(root, "model.bin")] + glob.glob(os.path.join(root, "*", "ids.i64")) +
                               glob.glob(os.path.join(root, "*", "exp_*.i32")) +
                               glob.glob(os.path.join(root, "*", "manifest.json"))) if os.path.exists(p))
    lines = [f"{sha256_file(p)}  {os.path.relpath(p, root)}" for p in names]
    if check:
        want = open(out).read().split("\n")
        bad = [l for l in lines if l not in want]
        for l in bad:
            print(f"{l.split('  ', 1)[1]}: FAILED")
        return 1 if bad or len(lines) != len([w for w in want if w]) else 0
    with open(out, "w") as f:
        f.write("\n".join(lines) + "\n")
    print(f"wrote {out} ({len(lines)} entries)")
    return 0


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("outdir")
    ap.add_argument("--config", choices=sorted(synth.CONFIGS))
    ap.add_argument("--seq", type=int, default=0, help="sequence of the config's batch")
    ap.add_argument("--ids", help="int64 little-endian token ids file")
    ap.add_argument("--window", type=int, default=0, help="label recorded in manifest.json")
    ap.add_argument("--model", help="model.bin (default: the synthetic model of the config)")
    ap.add_argument("--hash", action="store_true", help="write OUTDIR/vectors.sha256")
    ap.add_argument("--check", action="store_true", help="with --hash: verify instead of writing")
    a = ap.parse_args(argv)
    if a.hash:
        return hash_root(a.outdir, a.check)
    if bool(a.config) == bool(a.ids):
        ap.error("give exactly one of --config and --ids")
    if a.config:
        ids = synth.token_ids(a.config)[a.seq]
        window = synth.CONFIGS[a.config]["window"]
        model = a.model or synth.ensure_model("stress" if a.config == "cfg5" else "base")
    else:
        ids = np.fromfile(a.ids, dtype="<i8")
        window = a.window
        model = a.model or synth.ensure_model("base")
    man = export(a.outdir, ids, window, model)
    print("exported", {k: v["bytes"] for k, v in man["files"].items()})
    return 0


if __name__ == "__main__":
    sys.exit(main())
