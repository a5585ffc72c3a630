"""Real-weight path: model.bin and conformance vectors from the float SmolLM2-135M checkpoint.

    python -m eii.realweights MODEL_DIR OUTROOT [--data DATA_DIR]

MODEL_DIR holds model.safetensors (and tokenizer.json for the token windows), DATA_DIR
wikitext2_test.parquet — the assets python/fetch_assets.sh downloads at the pinned revision.
Writes OUTROOT/model.bin in the byte order of python/export_vectors.py:24-45: the weights
quantized by quant_rows / quant_vec_int16 (python/intref.py:113-130, eii/quant.py), the formats
of the scaling proposal in wide mode (eii/formats.py, python/intref.py:154-160), f_y = 8 and the
exp / RoPE / SiLU tables.  With --data it cuts the token windows as python/common.py:71-95 does
and exports, on the GPU, the three vector sets the reference pins (t24: window 64, 24 tokens;
t128: window 64, 128 tokens; t160: window 100, 160 tokens) and OUTROOT/vectors.sha256
(tools/hash_vectors.sh) — byte-identical to the reference's files when the assets are the
pinned ones.  The assets are not present offline, so the tests run the path on a synthetic
checkpoint of the same names and shapes.
"""
import argparse
import os
import sys

import numpy as np

from . import formats
from . import modelbin as mb
from . import tables
from .quant import quant_rows, quant_vec_int16

SEQ_LEN = 512                                   # python/common.py:24
SETS = (("t24", 64, 24), ("t128", 64, 128), ("t160", 100, 160))
F_Y = 8                                         # 15 - k(final_out | 30)


def _tensor_names(layer):
    p = f"model.layers.{layer}."
    return {"ln1": p + "input_layernorm.weight", "ln2": p + "post_attention_layernorm.weight",
            "q": p + "self_attn.q_proj.weight", "k": p + "self_attn.k_proj.weight",
            "v": p + "self_attn.v_proj.weight", "o": p + "self_attn.o_proj.weight",
            "gate": p + "mlp.gate_proj.weight", "up": p + "mlp.up_proj.weight",
            "down": p + "mlp.down_proj.weight"}


class Checkpoint:
    """Reads float tensors from model.safetensors as float32 numpy arrays (python/common.py:50-68:
    the stored dtype, bfloat16 for this model, converted to float32)."""

    def __init__(self, path):
        from safetensors import safe_open
        self.f = safe_open(path, framework="pt")

    def get(self, name):
        import torch
        return self.f.get_tensor(name).to(torch.float32).contiguous().numpy()


def build_model_bin(model_dir, out_path, log=print):
    """Quantize MODEL_DIR/model.safetensors into out_path (model.bin layout); returns out_path."""
    ck = Checkpoint(os.path.join(model_dir, "model.safetensors"))
    fm, f_y = formats.load_fm()
    assert f_y == F_Y
    emb_q, emb_m, emb_n = quant_rows(ck.get("model.embed_tokens.weight"))
    final_gain = quant_vec_int16(ck.get("model.norm.weight"))
    C, S = tables.rope_tables(mb.ROPE_POS)
    layers = []
    for l in range(mb.NL):
        names = _tensor_names(l)
        L = {"fm": np.asarray(fm[l], dtype=np.int64),
             "ln1": quant_vec_int16(ck.get(names["ln1"])), "ln2": quant_vec_int16(ck.get(names["ln2"]))}
        for m in mb.MATS:
            L[m] = quant_rows(ck.get(names[m]))
        f_g = int(fm[l][2 * mb.SITES.index("gate_proj") + 1])
        b_s, f_s = (int(v) for v in fm[l][2 * mb.SITES.index("silu_gate"):2 * mb.SITES.index("silu_gate") + 2])
        L["silu"] = tables.silu_table(f_g, f_s, b_s)
        layers.append(L)
        log(f"layer {l} quantized")
    mb.write(out_path, emb_q, emb_m, emb_n, final_gain, F_Y, tables.exp_table(), C, S, layers)
    return out_path


def token_windows(model_dir, data_dir):
    """Non-overlapping windows of SEQ_LEN tokens of the wikitext-2 raw test split, tokenized
    without special tokens (python/common.py:71-95)."""
    import pyarrow.parquet as pq
    from tokenizers import Tokenizer
    tok = Tokenizer.from_file(os.path.join(model_dir, "tokenizer.json"))
    rows = pq.read_table(os.path.join(data_dir, "wikitext2_test.parquet")).column("text").to_pylist()
    ids = tok.encode("\n\n".join(rows), add_special_tokens=False).ids
    n = len(ids) // SEQ_LEN
    return np.asarray(ids[: n * SEQ_LEN], dtype=np.int64).reshape(n, SEQ_LEN)


def export_sets(windows, model_path, outroot):
    """The reference's three vector sets from token windows [N, 512], computed on the GPU, and
    OUTROOT/vectors.sha256."""
    from . import export_vectors
    for name, win, T in SETS:
        export_vectors.export(os.path.join(outroot, name), windows[win][:T], win, model_path)
    model_link = os.path.join(outroot, "model.bin")
    if os.path.abspath(model_path) != os.path.abspath(model_link):
        if os.path.lexists(model_link):
            os.remove(model_link)
        os.symlink(os.path.abspath(model_path), model_link)
    return export_vectors.hash_root(outroot)


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("model_dir")
    ap.add_argument("outroot")
    ap.add_argument("--data", help="directory holding wikitext2_test.parquet: also export t24/t128/t160")
    a = ap.parse_args(argv)
    os.makedirs(a.outroot, exist_ok=True)
    path = build_model_bin(a.model_dir, os.path.join(a.outroot, "model.bin"))
    print(f"wrote {path}")
    if a.data:
        return export_sets(token_windows(a.model_dir, a.data), path, a.outroot)
    return 0


if __name__ == "__main__":
    sys.exit(main())
