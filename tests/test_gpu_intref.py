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


# every key python/intref.py:183,198-285 puts in a block trace
TRACE_KEYS = {"resid_in", "_f", "norm1_U", "norm1_z", "norm1_out", "q_proj", "k_proj", "v_proj", "q_rope",
              "k_rope", "attn_score", "attn_prob", "attn_ctx", "o_res", "resid_mid", "norm2_U", "norm2_z",
              "norm2_out", "gate_proj", "up_proj", "silu_gate", "mlp_gated", "down_res", "resid_out"}


@pytest.mark.parametrize("layer", [3, 11])
def test_embed_block_trace(M, oracle, layer):
    ids = synth.token_ids("cfg1")[0]
    x = M.embed(ids)
    assert np.array_equal(x, oracle.embed(ids))
    tr_g, tr_o = {}, {}
    y = M.block(layer, x, trace=tr_g)
    y_o = oracle.block(layer, x, len(ids), trace=tr_o)
    assert np.array_equal(y, y_o)
    assert set(tr_g) == TRACE_KEYS and set(tr_o) == TRACE_KEYS
    assert tr_g["_f"] == tr_o["_f"]
    T = len(ids)
    assert tr_g["attn_score"].shape == (9, T, T) and tr_g["attn_prob"].shape == (9, T, T)
    for k in TRACE_KEYS - {"_f"}:
        assert tr_g[k].dtype == np.int64, k
        assert np.array_equal(tr_g[k], np.asarray(tr_o[k]).reshape(tr_g[k].shape)), k
    # python/run_block.py:92-93 walks the format map and reads each named state
    for name, f in tr_g["_f"].items():
        assert tr_g[name].size > 0 and isinstance(f, int), name


def test_prop(M):
    """python/export_vectors.py:27,54 read prop["final_out|30"]["k"]; Model.fmt's rule gives the fm back."""
    assert 15 - M.prop["final_out|30"]["k"] == M.f_y == 8
    for l in (0, 11, 29):
        for site in ("norm1_out", "attn_ctx", "silu_gate", "mlp_gated"):
            e = M.prop[f"{site}|{l}"]
            flagged = e["class"].startswith("flagged")
            assert ((32, 31 - e["k"]) if flagged else (16, 15 - e["k"])) == M.fmt(site, l)


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


def test_matmul_any_k_and_int8(M):
    """matmul_exact for K off the multiples of 64 (zero-padded inside) and 8-bit activations."""
    import intref
    rng = np.random.default_rng(11)
    for K, bound in ((100, 1 << 7), (1000, 1 << 15), (3000, 1 << 31), (64, 1 << 7)):
        A = rng.integers(-bound, bound, size=(33, K)).astype(np.int64)
        A[0, :] = -bound
        A[1, :] = bound - 1
        W = rng.integers(-128, 128, size=(21, K)).astype(np.int64)
        W[0, :] = -128
        want = (A.astype(object) @ W.astype(object).T).astype(np.int64)
        got = intref.matmul_exact(A, W.astype(np.float64), bound, wmax=128 if bound < (1 << 31) else 127)
        assert np.array_equal(got, want), (K, bound)


def test_linear_wide_multiplier(M, oracle):
    """|m| above 2^14 and K off the model's shapes: the int64 requantization of python/intref.py:189."""
    rng = np.random.default_rng(12)
    for K, bits_in, mlo, mhi in ((576, 16, (1 << 14) + 1, (1 << 14) + 2), (200, 16, 1 << 20, 1 << 22),
                                 (576, 32, (1 << 14) + 1, (1 << 15))):
        a = rng.integers(-(1 << (bits_in - 1)), 1 << (bits_in - 1), size=(19, K)).astype(np.int64)
        q = rng.integers(-127, 128, size=(12, K)).astype(np.int8)
        m = rng.integers(mlo, mhi, size=12).astype(np.int64)
        n = rng.integers(30, 40, size=12).astype(np.int64)
        for f_in, f_out, bits_out in ((13, 10, 16), (13, 4, 32)):
            got, acc = M.linear(a, 1 << (bits_in - 1), (q, m, n), f_in, f_out, bits_out)
            want, acc_o = oracle.linear(a, 1 << (bits_in - 1), (q, m, n), f_in, f_out, bits_out)
            assert np.array_equal(acc, acc_o) and np.array_equal(got, want), (K, bits_in, mlo, f_out)


def test_rmsnorm_wide_gains(M, oracle):
    """Gains anywhere in int32 on the operator path: 3 z g formed in int64 and saturated before
    narrowing (c/intref.c:106-108), including the int16 ends and one-spike rows (|z| near 2^24)."""
    rng = np.random.default_rng(13)
    x = rng.integers(-2 ** 31, 2 ** 31, size=(40, 576)).astype(np.int64)
    x[:8] = 0
    for i in range(8):
        x[i, 7 * i] = (-1) ** i * (2 ** 31 - 1 - i)          # one spike: z reaches ~2^24
    for g in (np.full(576, 32767), np.full(576, -32768), np.where(np.arange(576) % 2, 32767, -32768),
              rng.integers(-2 ** 31 + 1, 2 ** 31, size=576), np.full(576, 50000), np.full(576, 2 ** 31 - 1)):
        g = g.astype(np.int64)
        for f_g, f_out, bits in ((14, 12, 16), (0, 11, 16), (14, 30, 32), (20, 0, 32), (3, 40, 32)):
            got = M.rmsnorm(x, (g, f_g), f_out, bits)
            want = oracle.rmsnorm(x, (g, f_g), f_out, bits)
            assert np.array_equal(got, want), (int(g[0]), f_g, f_out, bits)
