"""Real-weight path on the CPU (eii/quant.py, eii/realweights.py): float checkpoint -> model.bin.

The pinned SmolLM2-135M assets are absent offline, so a bfloat16 checkpoint with the same tensor
names and shapes (eii.synth.make_float_checkpoint) stands in for them.  Pins: hand-computed
quantizer cases; a per-row restatement with Python's math module (a different code path from
numpy) of quant_rows / quant_vec_int16 (python/intref.py:113-130) on rows of the stored model;
the model.bin layout (size, formats, tables); and the reference's own C checker accepting the
oracle's states on the built model."""
import math
import os
import subprocess

import numpy as np
import pytest

from eii import formats, realweights, synth, tables
from eii import modelbin as mb
from eii.quant import quant_rows, quant_vec_int16

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_BIN = os.path.join(ROOT, "oracle", "_ref", "intref")


def test_quant_rows_hand_cases():
    W = np.array([[127.0, -63.5, 0.0], [0.0, 0.0, 0.0], [127 * 2.0 ** -7, 1e-9, -0.5 * 2.0 ** -7]])
    q, m, n = quant_rows(W)
    assert q.tolist() == [[127, -64, 0], [0, 0, 0], [127, 0, 0]]   # rint: -63.5 -> -64, -0.5 -> -0
    assert m.tolist() == [8192, 8192, 8192] and n.tolist() == [13, 13, 20]


def test_quant_vec_int16_hand_cases():
    q, f = quant_vec_int16(np.array([1.0, -0.5, 0.25]))
    assert (q.tolist(), f) == ([16384, -8192, 4096], 14)
    q, f = quant_vec_int16(np.array([3.0, 1.5]))
    assert (q.tolist(), f) == ([24576, 12288], 13)


def _rows_by_math(W):
    """quant_rows restated row by row with the math module and Python's round (half to even)."""
    out = []
    for row in np.asarray(W, dtype=np.float64):
        s = max(abs(float(v)) for v in row) / 127.0
        s = 1.0 if s == 0 else s
        n = 13 - math.floor(np.log2(s))
        m = round(s * 2.0 ** n)
        step = m * 2.0 ** -n
        out.append(([max(-127, min(127, round(float(v) / step))) for v in row], m, n))
    return out


@pytest.fixture(scope="module")
def built(tmp_path_factory):
    d = tmp_path_factory.mktemp("ckpt")
    synth.make_float_checkpoint(str(d / "model.safetensors"), seed=3)
    realweights.build_model_bin(str(d), str(d / "model.bin"), log=lambda s: None)
    return d


def test_model_bin_layout(built):
    assert os.path.getsize(built / "model.bin") == mb.FILE_BYTES
    m = mb.read(str(built / "model.bin"))
    fm, f_y = formats.load_fm()
    assert m.f_y == f_y == 8
    assert np.array_equal(m.exp_tab, tables.exp_table())
    C, S = tables.rope_tables(mb.ROPE_POS)
    assert np.array_equal(m.rope_cos, C) and np.array_equal(m.rope_sin, S)
    for l in (0, 11, 29):
        assert np.array_equal(m.layers[l]["fm"], np.asarray(fm[l]))
        (_, f_g), (b_s, f_s) = m.fmt("gate_proj", l), m.fmt("silu_gate", l)
        assert np.array_equal(m.layers[l]["silu"], tables.silu_table(f_g, f_s, b_s))


def test_quantized_rows_match_math_restatement(built):
    ck = realweights.Checkpoint(str(built / "model.safetensors"))
    m = mb.read(str(built / "model.bin"))
    rng = np.random.default_rng(0)
    cases = [("model.embed_tokens.weight", m.emb_q, m.emb_m, m.emb_n)]
    for l, name, key in ((0, "q", "self_attn.q_proj"), (17, "gate", "mlp.gate_proj"), (29, "down", "mlp.down_proj")):
        q, mm, n = m.layers[l][name]
        cases.append((f"model.layers.{l}.{key}.weight", q, mm, n))
    for tname, q, mm, n in cases:
        W = ck.get(tname)
        rows = rng.choice(W.shape[0], size=6, replace=False)
        for r, (qr, mr, nr) in zip(rows, _rows_by_math(W[rows])):
            assert q[r].tolist() == qr and int(mm[r]) == mr and int(n[r]) == nr, (tname, r)
    g = ck.get("model.layers.5.input_layernorm.weight").astype(np.float64)
    f = 14 - math.floor(math.log2(max(abs(float(v)) for v in g)))
    assert m.layers[5]["ln1"][1] == f
    assert m.layers[5]["ln1"][0].tolist() == [max(-32768, min(32767, round(float(v) * 2.0 ** f))) for v in g]


@pytest.mark.skipif(not os.path.exists(REF_BIN), reason="oracle/_ref/intref not built (make -C oracle ref)")
def test_reference_checker_accepts_states_on_built_model(built, tmp_path):
    from oracle.intref_np import OracleModel, export_vectors
    ids = np.random.default_rng(9).integers(0, 49152, size=24, dtype=np.int64)
    export_vectors(OracleModel(str(built / "model.bin")), str(built), ids, str(tmp_path))
    r = subprocess.run([REF_BIN, str(tmp_path), str(built)], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0 and "ALL STATES EXACT" in r.stdout, r.stdout[-2000:]
