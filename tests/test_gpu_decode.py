"""Incremental decoding with a KV cache (eii_kv_*, eii_argmax).

The reference recomputes every position over the full prefix and names a cache as its next step,
to be tested by cached and uncached execution over the same fixed 32-token continuation and by a
greedy generation from the 128-token prompt (exact-integer-inference.tex:167).  Both are here:

* a 128-token prompt plus 32 single-token appends reproduces the committed golden digests of the
  full 160-token forward (which carry the reference C checker's ALL STATES EXACT verdict);
* appends in uneven chunks equal a full forward row for row;
* greedy generation with the cache follows the same trajectory as greedy generation by full
  forwards over the growing prefix;
* past the 160 positions the goldens cover, single-token steps at cache lengths 225..260 equal the
  numpy oracle's logits of the whole 260-token sequence.
"""
import hashlib
import json
import os

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from eii import synth
from eii import lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = json.load(open(os.path.join(ROOT, "tests", "golden", "golden.json")))


def sha(t):
    return hashlib.sha256(np.ascontiguousarray(t.cpu().numpy(), dtype=np.int32).tobytes()).hexdigest()


@pytest.fixture(scope="module")
def eng():
    from eii.engine import Engine
    e = Engine(synth.ensure_model("base"))
    yield e
    e.close()
    torch.cuda.empty_cache()


def test_prompt_plus_32_steps_matches_golden(eng):
    seqs = [37, 222]
    ids = torch.from_numpy(synth.token_ids("cfg4")[seqs]).to(eng.device)
    kv = eng.kv_cache(len(seqs), 160)
    try:
        parts = [kv.append(ids[:, :128])]
        for t in range(128, 160):
            parts.append(kv.append(ids[:, t:t + 1]))
        assert kv.length == 160
    finally:
        kv.close()
    lg = torch.cat(parts, dim=1)
    for i, s in enumerate(seqs):
        print(f"cfg4 sequence {s}", flush=True)
        assert sha(lg[i]) == GOLDEN["cfg4"]["sequences"][str(s)]["logits"]


@pytest.mark.parametrize("chunks", [[37, 1, 5, 32, 1, 24], [1] * 9 + [64, 31]])
def test_chunked_appends_equal_full_forward(eng, chunks):
    T = sum(chunks)
    ids = torch.from_numpy(np.random.default_rng(T).integers(0, 49152, size=(3, T), dtype=np.int64)).to(eng.device)
    full = eng.forward(ids)["logits"]
    kv = eng.kv_cache(3, T)
    try:
        t = 0
        for n in chunks:
            print(f"append {t}..{t + n - 1}", flush=True)
            lg = kv.append(ids[:, t:t + n])
            assert torch.equal(lg, full[:, t:t + n]), (t, n)
            t += n
    finally:
        kv.close()


@pytest.mark.parametrize("B", [4, 5])
def test_few_sequences_single_steps_equal_full_forward(eng, B):
    # single-token steps of up to 4 sequences fold the RMSNorm into the q/k/v, gate/up and head
    # GEMMs (a wave per row in their prologue); 5 sequences take the rmsnorm launches
    ids = torch.from_numpy(np.random.default_rng(40 + B).integers(0, 49152, size=(B, 44), dtype=np.int64)).to(eng.device)
    full = eng.forward(ids)["logits"]
    kv = eng.kv_cache(B, 44)
    try:
        kv.append(ids[:, :36], logits=False)
        for t in range(36, 44):
            lg = kv.append(ids[:, t:t + 1])
            assert torch.equal(lg[:, 0], full[:, t]), t
    finally:
        kv.close()


def test_many_sequences_single_steps_equal_full_forward(eng):
    # 96 sequences: the decoding attention runs one wave per head (few sequences take four)
    ids = torch.from_numpy(np.random.default_rng(96).integers(0, 49152, size=(96, 70), dtype=np.int64)).to(eng.device)
    full = eng.forward(ids)["logits"]
    kv = eng.kv_cache(96, 70)
    try:
        kv.append(ids[:, :64], logits=False)
        for t in range(64, 70):
            lg = kv.append(ids[:, t:t + 1])
            assert torch.equal(lg[:, 0], full[:, t]), t
    finally:
        kv.close()


def test_long_context_single_steps_equal_full_forward():
    # single-token steps at cache lengths from 291 to 8194 on the stress model (q/k saturate, so
    # many keys fall beyond the exp table): lengths up to 8192 take the one-query decoding
    # kernel, longer ones the tiled attention; each step's logits equal the full forward's row
    from eii.engine import Engine
    T = 8194
    e = Engine(synth.ensure_model("stress"), rope_rows=T)
    try:
        ids = torch.from_numpy(np.random.default_rng(8).integers(0, 49152, size=(2, T), dtype=np.int64)).to(e.device)
        full = e.forward(ids)["logits"]
        kv = e.kv_cache(2, T)
        try:
            t = 0
            for start, steps in ((290, 3), (1029, 2), (8190, 4)):
                print(f"append {t}..{start - 1}, then {steps} single steps", flush=True)
                kv.append(ids[:, t:start], logits=False)
                t = start
                for _ in range(steps):
                    lg = kv.append(ids[:, t:t + 1])
                    assert torch.equal(lg[:, 0], full[:, t]), t
                    t += 1
        finally:
            kv.close()
    finally:
        del full
        e.close()
        torch.cuda.empty_cache()


def test_steps_past_160_positions_match_oracle(eng):
    # a 224-token prompt (tiled attention), then 36 single-token steps (the one-query decoding
    # kernel over 225..260 cached positions), each step's logits against the oracle's row
    from oracle.intref_np import OracleModel
    T, P = 260, 224
    ids_np = np.random.default_rng(260).integers(0, 49152, size=(1, T), dtype=np.int64)
    print("oracle forward over 260 positions (about 20 s of CPU)", flush=True)
    want = OracleModel(synth.ensure_model("base"), rope_rows=T).forward(ids_np)[2][0]
    ids = torch.from_numpy(ids_np).to(eng.device)
    kv = eng.kv_cache(1, T)
    try:
        lg = kv.append(ids[:, :P])
        assert np.array_equal(lg[0].cpu().numpy(), want[:P])
        for t in range(P, T):
            lg = kv.append(ids[:, t:t + 1])
            assert np.array_equal(lg[0, 0].cpu().numpy(), want[t]), t
    finally:
        kv.close()


def test_greedy_trajectory_cached_equals_recomputed(eng):
    prompt = torch.from_numpy(synth.token_ids("cfg4")[[0, 111], :128]).to(eng.device)
    toks, lg = eng.generate(prompt, 32)
    assert toks.shape == (2, 32) and lg.shape == (2, 159, 49152)
    seq = prompt
    for i in range(32):
        full = eng.forward(seq)["logits"]
        nxt = eng.argmax(full[:, -1])
        assert torch.equal(nxt, toks[:, i]), i
        seq = torch.cat([seq, nxt[:, None]], dim=1)
    assert torch.equal(full, lg)   # the last recomputation covers positions 0..158


def test_argmax_ties_and_numpy_rule(eng):
    rng = np.random.default_rng(5)
    a = rng.integers(-3, 3, size=(7, 49152)).astype(np.int32)   # many equal maxima
    a[1] = 7
    a[2] = np.iinfo(np.int32).min
    a[3, 49151] = 2 ** 31 - 1
    t = torch.from_numpy(a).to(eng.device)
    assert eng.argmax(t).cpu().numpy().tolist() == np.argmax(a, axis=1).tolist()


def test_kv_bounds_and_reset(eng):
    ids = torch.zeros((2, 40), dtype=torch.int64, device=eng.device)
    kv = eng.kv_cache(2, 40)   # capacity rounds up to 64 positions
    try:
        kv.append(ids[:, :40], logits=False)
        kv.append(ids[:, :24], logits=False)
        assert kv.length == 64
        with pytest.raises(L.EIIError) as e:
            kv.append(ids[:, :1], logits=False)
        assert e.value.code == L.EII_E_BOUND
        with pytest.raises(L.EIIError) as e:
            kv.append(ids[:1, :1], logits=False)
        assert e.value.code == L.EII_E_ARG
        kv.reset()
        assert kv.length == 0
        lg = kv.append(ids[:, :3])
        assert torch.equal(lg, eng.forward(ids[:, :3])["logits"])
    finally:
        kv.close()
