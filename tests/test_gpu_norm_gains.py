"""The forward's RMSNorm kernel (int16 gains, fast int32 path) at the ends of the int16 gain range:
a model.bin whose layer-0 gains sit at -32768 and 32767, against the oracle (python/intref.py:168-184).
A gain outside int16 is rejected at load (tests/test_abi.py)."""
import shutil

import numpy as np
import pytest
import torch

from eii import modelbin, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def extreme_model(tmp_path_factory, model_path):
    p = tmp_path_factory.mktemp("gains") / "model_extreme_gains.bin"
    shutil.copyfile(model_path, p)
    g1 = np.where(np.arange(576) % 3 == 0, -32768, 32767).astype("<i8")
    g2 = np.where(np.arange(576) % 2 == 0, 32767, -32768).astype("<i8")
    base = modelbin.HEADER_BYTES + 24 * 8
    with open(p, "r+b") as f:
        f.seek(base)
        f.write(g1.tobytes())                 # ln1 of layer 0
        f.seek(base + 576 * 8 + 8)
        f.write(g2.tobytes())                 # ln2 of layer 0
        f.seek(49152 * 576 + 2 * 49152 * 8)
        f.write(np.full(576, -32768, dtype="<i8").tobytes())   # final gain
    return str(p)


def test_extreme_int16_gains(extreme_model):
    from eii.engine import Engine
    from oracle.intref_np import OracleModel
    ora = OracleModel(extreme_model)
    eng = Engine(extreme_model)
    try:
        ids = synth.token_ids("cfg1")[0]
        x0 = ora.embed(ids)
        x0[:3] = 0
        x0[0, 5] = 2 ** 31 - 1                 # one-spike rows: |z| reaches 2^24
        x0[1, 9] = -2 ** 31
        x0[2, 100] = 123456789
        x = torch.from_numpy(x0.astype(np.int32)).cuda()
        tr = eng.block(0, x, 1, len(ids), trace=True)
        want = {}
        xo = ora.block(0, x0, len(ids), want)
        for k in ("norm1_out", "norm1_U", "norm1_z", "norm2_out", "norm2_U", "norm2_z"):
            got = tr[k].cpu().numpy().astype(np.int64).reshape(want[k].shape)
            assert np.array_equal(got, want[k]), k
        assert np.array_equal(x.cpu().numpy().astype(np.int64), xo)
        lg = eng.final(x).cpu().numpy().astype(np.int64)
        assert np.array_equal(lg, ora.final(xo))
    finally:
        eng.close()


@pytest.fixture(scope="module")
def left_shift_model(tmp_path_factory, model_path):
    """Layer 0's ln1 exponent lowered so the norm's output shift is -25: a left shift by 25 of values up
    to 2^41, which wraps in the reference's int64 (the kernel's int64 path below shift -21)."""
    p = tmp_path_factory.mktemp("lshift") / "model_norm_lshift.bin"
    shutil.copyfile(model_path, p)
    f_norm1 = int(modelbin.read(model_path).layers[0]["fm"][1])
    with open(p, "r+b") as f:
        f.seek(modelbin.HEADER_BYTES + 24 * 8 + 576 * 8)
        f.write(np.array([-25 - 21 + f_norm1], dtype="<i8").tobytes())
    return str(p)


def test_norm_left_shift_wraps_like_int64(left_shift_model):
    from eii.engine import Engine
    from oracle.intref_np import OracleModel
    ora = OracleModel(left_shift_model)
    eng = Engine(left_shift_model)
    try:
        ids = synth.token_ids("cfg1")[0]
        x0 = ora.embed(ids)
        x = torch.from_numpy(x0.astype(np.int32)).cuda()
        tr = eng.block(0, x, 1, len(ids), trace=True)
        want = {}
        ora.block(0, x0, len(ids), want)
        for k in ("norm1_out", "norm1_U", "norm1_z"):
            got = tr[k].cpu().numpy().astype(np.int64).reshape(want[k].shape)
            assert np.array_equal(got, want[k]), k
    finally:
        eng.close()
