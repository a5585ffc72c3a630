"""The python/intref.py drop-in (exact-integer-inference_amd/intref.py) against the oracle."""
import numpy as np
import pytest

from eii import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def M(model_path):
    import intref
    return intref.Model(model_bin=model_path)


def test_forward_matches_oracle(M, oracle):
    ids = synth.token_ids("cfg1")[0]
    _, _, lg = oracle.forward(ids[None, :])
    got = M.forward(ids)
    assert got.dtype == np.int64 and got.shape == (24, 49152)
    assert np.array_equal(got, lg[0])


def test_embed_block_trace(M, oracle):
    ids = synth.token_ids("cfg1")[0]
    x = M.embed(ids)
    assert np.array_equal(x, oracle.embed(ids))
    tr_g, tr_o = {}, {}
    y = M.block(3, x, trace=tr_g)
    y_o = oracle.block(3, x, len(ids), trace=tr_o)
    assert np.array_equal(y, y_o)
    for k in ("norm1_out", "q_proj", "k_proj", "v_proj", "q_rope", "k_rope", "attn_ctx", "resid_mid",
              "norm2_out", "gate_proj", "up_proj", "mlp_gated", "resid_in", "resid_out"):
        assert np.array_equal(tr_g[k], tr_o[k]), k


def test_operators(M, oracle):
    import intref
    rng = np.random.default_rng(3)
    x = rng.integers(-2 ** 31, 2 ** 31, size=(37, 576)).astype(np.int64)
    g = M.layers[5]["ln2"]
    assert np.array_equal(M.rmsnorm(x, g, 12, 16), oracle.rmsnorm(x, g, 12, 16))
    a = rng.integers(-2 ** 15, 2 ** 15, size=(45, 576)).astype(np.int64)
    W = M.layers[7]["gate"]
    out, acc = M.linear(a, 1 << 15, W, 13, 10, 16)
    out_o, acc_o = oracle.linear(a, 1 << 15, W, 13, 10, 16)
    assert np.array_equal(acc, acc_o) and np.array_equal(out, out_o)
    A = rng.integers(-2 ** 31, 2 ** 31, size=(9, 1536)).astype(np.int64)
    Wq = M.layers[2]["down"][0]
    want = (A.astype(object) @ Wq.astype(object).T).astype(np.int64)
    assert np.array_equal(intref.matmul_exact(A, Wq.astype(np.float64), 1 << 31), want)
    assert M.fmt("attn_ctx", 0) == (32, 30) and M.fmt("final_out", 30) == (16, 8)
