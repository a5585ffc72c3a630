"""Operator parity of the HIP kernels with the oracle (exact integer equality)."""
import ctypes as C

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from eii import lib as L
from eii.tables import exp_table


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def p(t):
    return C.c_void_p(t.data_ptr())


def gemm(A, W):
    lib = L.load()
    a_bits = 16 if A.dtype == np.int16 else 32
    M, K = A.shape
    N = W.shape[0]
    acc = torch.empty((M, N), dtype=torch.int64, device="cuda")
    At, Wt = dev(A), dev(W)                          # keep the inputs alive until the kernel ran
    L.check(lib.eii_gemm_i8(p(At), a_bits, p(Wt), M, N, K, p(acc), None))
    torch.cuda.synchronize()
    return acc.cpu().numpy()


def exact_mm(A, W):
    # float64 BLAS is exact while K * max|a| * 127 < 2^53 (python/intref.py:58-63)
    assert A.shape[1] * 2.0 ** 31 * 127 < 2.0 ** 53
    return np.rint(A.astype(np.float64) @ W.astype(np.float64).T).astype(np.int64)


@pytest.mark.parametrize("a_dtype", [np.int16, np.int32])
@pytest.mark.parametrize("M,N,K", [(1, 16, 64), (197, 80, 128), (130, 200, 576), (64, 576, 1536)])
def test_gemm_small(a_dtype, M, N, K):
    rng = np.random.default_rng(M * 1000 + N + K)
    info = np.iinfo(a_dtype)
    A = rng.integers(info.min, info.max, size=(M, K), endpoint=True, dtype=np.int64).astype(a_dtype)
    A[0, :4] = [info.min, info.max, -1, 0]
    W = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    W[0, :3] = [-128, 127, -1]                       # the full int8 range, beyond model weights
    got = gemm(A, W)
    np.testing.assert_array_equal(got, exact_mm(A, W))


def test_gemm_staging_two_streams():
    # the operator entry points share one staging block per device: calls alternating between
    # two streams, with sizes that grow (a new block) and shrink (the old one reused), are
    # ordered by the block's event and each gives its own exact result
    lib = L.load()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    cases = []
    for i, (M, N, K, dt) in enumerate([(64, 80, 576, np.int16), (900, 576, 1536, np.int32), (33, 192, 576, np.int32),
                                       (2000, 960, 576, np.int16), (5, 16, 64, np.int16), (700, 200, 128, np.int32)]):
        rng = np.random.default_rng(100 + i)
        info = np.iinfo(dt)
        A = rng.integers(info.min, info.max, size=(M, K), endpoint=True, dtype=np.int64).astype(dt)
        W = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
        At, Wt = dev(A), dev(W)
        acc = torch.empty((M, N), dtype=torch.int64, device="cuda")
        cases.append((A, W, At, Wt, acc))
    torch.cuda.synchronize()
    for i, (A, W, At, Wt, acc) in enumerate(cases):
        s = streams[i % 2]
        M, K = A.shape
        L.check(lib.eii_gemm_i8(p(At), 16 if A.dtype == np.int16 else 32, p(Wt), M, W.shape[0], K, p(acc),
                                C.c_void_p(s.cuda_stream)))
    torch.cuda.synchronize()
    for A, W, At, Wt, acc in cases:
        np.testing.assert_array_equal(acc.cpu().numpy(), exact_mm(A, W))


def test_gemm_layout_probe():
    # one-hot rows and columns: acc[m, n] picks single products, so a wrong lane/byte layout of
    # the MFMA operands shows up as a misplaced entry rather than a different sum
    M, N, K = 64, 64, 64
    A = np.zeros((M, K), dtype=np.int16)
    W = np.zeros((N, K), dtype=np.int8)
    for m in range(M):
        A[m, (5 * m + 3) % K] = 1000 + m
    for n in range(N):
        W[n, (5 * n + 3) % K] = 1 + (n % 100)
    got = gemm(A, W)
    np.testing.assert_array_equal(got, exact_mm(A, W))


def test_rmsnorm(oracle):
    lib = L.load()
    rng = np.random.default_rng(7)
    x = rng.integers(-2 ** 31, 2 ** 31, size=(37, 576), dtype=np.int64)
    x[1] = -2 ** 31                                  # largest sum of squares
    x[2] = 0                                         # only epsilon
    x[3] = rng.integers(-3, 4, size=576)
    x[4, :] = 0; x[4, 7] = 2 ** 31 - 1               # one element carries everything
    x[5] = rng.integers(-2 ** 16, 2 ** 16, size=576)
    gain = rng.integers(-2 ** 15, 2 ** 15, size=576, dtype=np.int64)
    xt, gt = dev(x.astype(np.int32)), dev(gain.astype(np.int32))
    # shifts 22, 24, 13, 10 (fast path edge), -5, 7 and 41 (general path)
    for f_gain, f_out, bits in [(14, 13, 16), (14, 11, 16), (12, 20, 32), (14, 25, 32), (14, 40, 16), (14, 28, 32),
                                (20, 0, 16)]:
        want = oracle.rmsnorm(x, (gain, f_gain), f_out, bits)
        out = torch.empty((37, 576), dtype=torch.int16 if bits == 16 else torch.int32, device="cuda")
        L.check(lib.eii_rmsnorm(p(xt), 37, p(gt), f_gain, f_out, bits, p(out), None))
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out.cpu().numpy().astype(np.int64), want)


@pytest.mark.parametrize("f_q,f_qr,bits_qr,f_k,f_kr,bits_kr", [
    (10, 11, 16, 9, 9, 16),       # shifts 29 and 30
    (10, 13, 16, 9, 12, 16),      # shifts 27: the rotated values saturate
    (12, 11, 12, 9, 10, 10),      # narrower outputs
    (2, 40, 16, 9, 45, 16),       # shifts -8 and -6: exact left shifts, saturating
])
def test_rope_operator(oracle, f_q, f_qr, bits_qr, f_k, f_kr, bits_kr):
    # python/intref.py:212-225 on packed sequences: positions restart at 0 in each sequence
    lib = L.load()
    lens = [5, 160, 33, 1]
    M = sum(lens)
    rng = np.random.default_rng(f_qr * 100 + bits_qr)
    qkv = rng.integers(-32768, 32768, size=(M, 960), dtype=np.int64)
    qkv[0, :4] = [-32768, 32767, 0, -1]
    qkv[1, 32:36] = [-32768, 32767, -32768, 32767]
    off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    qt, ot = dev(qkv.astype(np.int16)), dev(off)
    ct, st = dev(oracle.rope_c.astype(np.int32)), dev(oracle.rope_s.astype(np.int32))
    L.check(lib.eii_rope(p(qt), p(ot), len(lens), p(ct), p(st), oracle.rope_c.shape[0], f_q, f_qr, bits_qr, f_k, f_kr,
                         bits_kr, None))
    torch.cuda.synchronize()
    got = qt.cpu().numpy().astype(np.int64)
    pos = np.concatenate([np.arange(T) for T in lens])
    np.testing.assert_array_equal(got[:, :576].reshape(M, 9, 64), oracle.rope(qkv[:, :576], 9, pos, f_q, f_qr, bits_qr))
    np.testing.assert_array_equal(got[:, 576:768].reshape(M, 3, 64),
                                  oracle.rope(qkv[:, 576:768], 3, pos, f_k, f_kr, bits_kr))
    np.testing.assert_array_equal(got[:, 768:], qkv[:, 768:])   # v untouched


def test_rope_operator_rows_bound(oracle):
    lib = L.load()
    qt = torch.zeros((600, 960), dtype=torch.int16, device="cuda")
    ot = dev(np.array([0, 600], dtype=np.int32))
    ct = dev(oracle.rope_c.astype(np.int32))
    assert lib.eii_rope(p(qt), p(ot), 1, p(ct), p(ct), oracle.rope_c.shape[0], 10, 11, 16, 9, 9, 16, None) == \
        L.EII_E_BOUND


@pytest.mark.parametrize("f_g,f_s,bits_s,f_u,f_m,bits_m", [
    (12, 13, 16, 12, 12, 16),     # shift 13
    (10, 13, 16, 12, 25, 32),     # shift 0
    (13, 14, 32, 11, 30, 32),     # 32-bit table, shift -5
    (11, 13, 16, 12, 5, 16),      # shift 20
    (9, 14, 16, 14, 14, 16),      # saturating products
])
def test_silu_gate_operator(f_g, f_s, bits_s, f_u, f_m, bits_m):
    from eii.tables import silu_table
    from oracle.intref_np import silu_gate
    lib = L.load()
    M = 37
    rng = np.random.default_rng(f_m * 10 + bits_s)
    g = rng.integers(-32768, 32768, size=(M, 1536), dtype=np.int64)
    u = rng.integers(-32768, 32768, size=(M, 1536), dtype=np.int64)
    g[0, :3] = [-32768, 32767, 0]
    u[0, :3] = [-32768, -32768, 32767]
    u[1, :] = 0
    tab = np.asarray(silu_table(f_g, f_s, bits_s), dtype=np.int64)
    out = torch.empty((M, 1536), dtype=torch.int16 if bits_m == 16 else torch.int32, device="cuda")
    gt, ut, tt = dev(g.astype(np.int16)), dev(u.astype(np.int16)), dev(tab.astype(np.int32))
    L.check(lib.eii_silu_gate(p(gt), p(ut), M, p(tt), f_s, f_u, f_m, bits_m, p(out), None))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy().astype(np.int64), silu_gate(tab, g, u, f_s, f_u, f_m, bits_m))


def _attention_case(oracle, lens, scale, seed, f_qr=10, f_kr=9, f_v=11, f_c=11, bits_c=16, floor=False):
    lib = L.load()
    rng = np.random.default_rng(seed)
    M = sum(lens)
    qkv = np.clip(np.round(rng.standard_normal((M, 960)) * scale), -32768, 32767).astype(np.int16)
    if floor:   # q >= 0 and k <= 0: every q.k is far below zero
        qkv[:, :576] = np.minimum(np.abs(qkv[:, :576].astype(np.int64)), 32767)
        qkv[:, 576:768] = -np.minimum(np.abs(qkv[:, 576:768].astype(np.int64)), 32767)
    off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    E = exp_table().astype(np.int32)
    ctx = torch.empty((M, 576), dtype=torch.int16 if bits_c == 16 else torch.int32, device="cuda")
    qt, ot, et = dev(qkv), dev(off), dev(E)
    L.check(lib.eii_attention(p(qt), p(ot), len(lens), max(lens), p(et), f_qr, f_kr, f_v, f_c, bits_c, p(ctx),
                              None))
    torch.cuda.synchronize()
    got = ctx.cpu().numpy().astype(np.int64)
    shift_s = f_qr + f_kr + 3 - 7
    q = qkv[:, :576].astype(np.int64).reshape(M, 9, 64)
    k = qkv[:, 576:768].astype(np.int64).reshape(M, 3, 64)
    v = qkv[:, 768:].astype(np.int64).reshape(M, 3, 64)
    for b in range(len(lens)):
        sl = slice(off[b], off[b + 1])
        want = oracle.attention(q[sl], k[sl], v[sl], shift_s, f_v, f_c, bits_c, 16, 16, 16)
        np.testing.assert_array_equal(got[sl], want.reshape(-1, 576), err_msg=f"sequence {b}")


@pytest.mark.parametrize("scale", [300.0, 2000.0])
@pytest.mark.parametrize("lens", [[1], [64], [65, 3, 130], [160, 160]])
def test_attention_spread(oracle, lens, scale):
    _attention_case(oracle, lens, scale=scale, seed=len(lens))


def test_attention_saturated(oracle):
    # scores pinned at the 16-bit limits: many keys fall beyond the table (d > 1536), P = 65536 occurs
    _attention_case(oracle, [150, 7], scale=20000.0, seed=3, f_qr=8, f_kr=8)


@pytest.mark.parametrize("lens", [[150, 7], [33, 200], [64, 96], [45, 300]])
def test_attention_scores_at_floor(oracle, lens):
    # every score saturates at -32768: the row max is -32768, so a masked key (score -32768) would
    # fall inside the exp table; the tiles holding masked keys must test them
    _attention_case(oracle, lens, scale=20000.0, seed=11 + len(lens), f_qr=8, f_kr=8, floor=True)


@pytest.mark.parametrize("nseq,lo,hi", [(40, 130, 161), (24, 200, 251)])
def test_attention_large_batches(oracle, nseq, lo, hi):
    # many ragged sequences (starts off the 32-row tile grid) in one launch, up to 5 and up to 8
    # key tiles
    lens = list(np.random.default_rng(nseq).integers(lo, hi, size=nseq))
    _attention_case(oracle, lens, scale=2000.0, seed=nseq)
    _attention_case(oracle, lens, scale=20000.0, seed=nseq + 1, f_qr=8, f_kr=8, floor=True)


def test_attention_ctx32(oracle):
    _attention_case(oracle, [100], scale=3000.0, seed=5, f_c=27, bits_c=32)


@pytest.mark.parametrize("lens", [[33, 200], [45, 300], [700]])
def test_attention_long(oracle, lens):
    # sequences over 8 key tiles take the variant that recomputes scores per pass; starts that
    # are not multiples of 32 exercise the masked first key tile
    _attention_case(oracle, lens, scale=2000.0, seed=sum(lens))
    _attention_case(oracle, lens, scale=20000.0, seed=sum(lens) + 1, f_qr=8, f_kr=8)


@pytest.mark.parametrize("a_bits,out_bits,M,N,K", [(16, 16, 300, 192, 576), (16, 32, 37, 576, 576),
                                                    (32, 16, 130, 576, 1536), (32, 32, 64, 1536, 576),
                                                    (16, 16, 257, 3072, 576)])
def test_linear_requant(oracle, a_bits, out_bits, M, N, K):
    # python/intref.py:186-190 on random operands, including the extreme activation values and
    # multipliers at both ends of [2^13, 2^14]; shifts near their smallest and largest values
    lib = L.load()
    rng = np.random.default_rng(a_bits * 7 + out_bits + M)
    lim = 2 ** (a_bits - 1)
    a = rng.integers(-lim, lim, size=(M, K), dtype=np.int64)
    a[0, :] = -lim
    a[1, :] = lim - 1
    a[2, :] = rng.integers(-3, 4, size=K)
    W = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    W[:, 0] = 127
    m = rng.integers(2 ** 13, 2 ** 14 + 1, size=N, dtype=np.int64)
    m[:2] = [2 ** 13, 2 ** 14]
    n = rng.integers(18, 30, size=N, dtype=np.int64)
    n[2:6] = [10, 11, 44, 45]
    f_in, f_out = 12, 9
    want, _ = oracle.linear(a, lim, (W, m, n), f_in, f_out, out_bits)
    at = dev(a.astype(np.int16 if a_bits == 16 else np.int32))
    wt = dev(W)
    ws = torch.empty(N, dtype=torch.int32, device="cuda")
    mt = dev(m.astype(np.int32))
    st = dev((n + f_in - f_out).astype(np.int32))
    out = torch.empty((M, N), dtype=torch.int16 if out_bits == 16 else torch.int32, device="cuda")
    L.check(lib.eii_weight_colsum(p(wt), N, K, p(ws), None))
    L.check(lib.eii_linear(p(at), a_bits, p(wt), p(ws), p(mt), p(st), M, N, K, out_bits, p(out), None))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy().astype(np.int64), want)
