"""Data-dependent violations on the GPU: the conditions the reference asserts (an embedding index
outside the vocabulary, python/intref.py:163-166 through numpy indexing; a logit outside int32,
python/export_vectors.py:58) are reported by eii_check as status 4 (EII_E_BOUND), and a later
clean call succeeds again."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from eii import lib as L
from eii import modelbin as mb
from eii import synth
from oracle.intref_np import OracleModel


def test_token_id_outside_vocabulary(engine):
    ids = synth.token_ids("cfg1")[:1].copy()
    for bad in (49152, -1):
        ids[0, 5] = bad
        with pytest.raises(L.EIIError) as e:
            engine.forward(ids, logits=False)
        assert e.value.code == L.EII_E_BOUND
    engine.forward(synth.token_ids("cfg1")[:1], logits=False)   # the report was cleared


def _head_model(tmp_path, n0):
    """The synthetic model with vocabulary row 0 all 127 (m = 2^14, n = n0) and a final gain of
    32767 at f = 7: an all-equal positive residual saturates every normalized value at 32767, so
    logit 0 is 32767 * 127 * 576 * 2^14 / 2^(n0 - 8), past int32 for n0 = 16."""
    m = mb.read(synth.ensure_model("base"))
    emb_q, emb_m, emb_n = np.array(m.emb_q), np.array(m.emb_m), np.array(m.emb_n)
    emb_q[0] = 127
    emb_m[0] = 2 ** 14
    emb_n[0] = n0
    gain = (np.full(576, 32767, dtype=np.int64), 7)
    path = tmp_path / f"head_{n0}.bin"
    mb.write(str(path), emb_q, emb_m, emb_n, gain, m.f_y, m.exp_tab, m.rope_cos, m.rope_sin, m.layers)
    return str(path)


@pytest.mark.parametrize("n0,overflow", [(16, True), (30, False)])
def test_logit_outside_int32(tmp_path, n0, overflow):
    from eii.engine import Engine
    path = _head_model(tmp_path, n0)
    x = np.full((4, 576), 2 ** 20, dtype=np.int64)
    x[1] = 1 << 30
    x[2, ::2] = -(1 << 25)
    eng = Engine(path)
    try:
        xt = torch.from_numpy(x.astype(np.int32)).to(eng.device)
        if overflow:
            with pytest.raises(L.EIIError) as e:
                eng.final(xt)
            assert e.value.code == L.EII_E_BOUND
        else:
            got = eng.final(xt).cpu().numpy().astype(np.int64)
            want = OracleModel(path).final(x)
            assert np.abs(want[:, 0]).max() > 2 ** 20   # large, inside int32
            np.testing.assert_array_equal(got, want)
    finally:
        eng.close()
        torch.cuda.empty_cache()
