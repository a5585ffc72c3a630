"""Forward parity of the HIP engine with the oracle: every residual and every logit exact."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from eii import synth

SITES16 = ("norm1_out", "q_proj", "k_proj", "v_proj", "q_rope", "k_rope", "attn_ctx", "norm2_out",
           "gate_proj", "up_proj", "mlp_gated")


def first_diff(got, want):
    bad = np.flatnonzero(got.reshape(-1) != want.reshape(-1))
    if bad.size == 0:
        return None
    i = bad[0]
    return f"{bad.size} of {got.size} differ, first at {i} (got {got.reshape(-1)[i]} expected {want.reshape(-1)[i]})"


def test_embed(engine, oracle):
    ids = synth.token_ids("cfg1")[0]
    got = engine.embed(ids).cpu().numpy().astype(np.int64)
    assert first_diff(got, oracle.embed(ids)) is None


@pytest.mark.parametrize("layer", [0, 4, 11, 28])
def test_block_trace(engine, oracle, layer):
    ids = synth.token_ids("cfg1")[0]
    x0 = oracle.embed(ids)
    x = torch.from_numpy(x0.astype(np.int32)).cuda()
    tr = engine.block(layer, x, 1, len(ids), trace=True)
    torch.cuda.synchronize()
    want = {}
    xo = oracle.block(layer, x0, len(ids), want)
    for s in SITES16 + ("resid_mid",):
        msg = first_diff(tr[s].cpu().numpy().astype(np.int64), want[s].reshape(len(ids), -1))
        assert msg is None, f"layer {layer} site {s}: {msg}"
    assert first_diff(x.cpu().numpy().astype(np.int64), xo) is None


def test_forward_cfg1(engine, oracle):
    ids = synth.token_ids("cfg1")
    out = engine.forward(ids, embed=True, resid=True, logits=True)
    emb, res, lg = oracle.forward(ids)
    assert first_diff(out["embed"].cpu().numpy(), emb) is None
    got_res = out["resid"].cpu().numpy()
    for l in range(30):
        msg = first_diff(got_res[l], res[l])
        assert msg is None, f"layer {l}: {msg}"
    assert first_diff(out["logits"].cpu().numpy(), lg) is None


def test_forward_dump_selection(engine):
    # the states of selected sequences, packed in batch order, equal their rows of a full dump;
    # logits always cover the whole batch
    rng = np.random.default_rng(12)
    ids = rng.integers(0, 49152, size=(5, 40), dtype=np.int64)
    full = engine.forward(ids, embed=True, resid=True, logits=True)
    for sel in ([3], [0, 1, 4], [4, 2]):
        part = engine.forward(ids, embed=True, resid=True, logits=True, dump=sel)
        order = sorted(sel)
        assert torch.equal(part["embed"], full["embed"][order])
        assert torch.equal(part["resid"], full["resid"][:, order])
        assert torch.equal(part["logits"], full["logits"])
    lens = [7, 33, 1, 20]
    flat = rng.integers(0, 49152, size=sum(lens), dtype=np.int64)
    fullp = engine.forward_packed(flat, lens, embed=True, resid=True)
    part = engine.forward_packed(flat, lens, embed=True, resid=True, dump=[1, 2])
    assert torch.equal(part["embed"], fullp["embed"][7:41])
    assert torch.equal(part["resid"], fullp["resid"][:, 7:41])
    assert torch.equal(part["logits"], fullp["logits"])


def test_forward_ragged_batch(engine, oracle):
    # sequences of different lengths packed in one forward equal their own B=1 runs
    rng = np.random.default_rng(11)
    lens = [24, 1, 70, 9]
    ids = [rng.integers(0, 49152, size=t, dtype=np.int64) for t in lens]
    out = engine.forward_packed(np.concatenate(ids), lens, resid=True, logits=True)
    res = out["resid"].cpu().numpy()
    lg = out["logits"].cpu().numpy()
    off = np.concatenate([[0], np.cumsum(lens)])
    for b, t in enumerate(lens):
        _, r1, l1 = oracle.forward(ids[b][None, :])
        sl = slice(off[b], off[b + 1])
        assert first_diff(res[:, sl], r1[:, 0]) is None, f"sequence {b}"
        assert first_diff(lg[sl], l1[0]) is None, f"sequence {b}"


@pytest.mark.parametrize("lens", [[3], [2, 1, 1]])
def test_forward_few_rows(engine, oracle, lens):
    # at most 4 rows: the q/k/v, gate/up and head GEMMs form the RMSNorm in their prologue (a
    # plain forward, so the q/k/v epilogue also writes the V^T planes); every residual and logit
    # against the oracle's runs of each sequence
    rng = np.random.default_rng(3 + len(lens))
    ids = [rng.integers(0, 49152, size=t, dtype=np.int64) for t in lens]
    out = engine.forward_packed(np.concatenate(ids), lens, resid=True, logits=True)
    res = out["resid"].cpu().numpy()
    lg = out["logits"].cpu().numpy()
    off = np.concatenate([[0], np.cumsum(lens)])
    for b, t in enumerate(lens):
        _, r1, l1 = oracle.forward(ids[b][None, :])
        sl = slice(off[b], off[b + 1])
        assert first_diff(res[:, sl], r1[:, 0]) is None, f"sequence {b}"
        assert first_diff(lg[sl], l1[0]) is None, f"sequence {b}"
