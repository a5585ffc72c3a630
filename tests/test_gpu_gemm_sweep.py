"""The exact matmul (python/intref.py:58-63) at the projection shapes with M = 4096 rows of int32
and int16 activations, 1 % of them anywhere in the type's range: every row of the four smaller
shapes against float64 BLAS (exact: K * 2^31 * 127 < 2^53), and for the 576 x 49152 head shape
512 sampled rows plus the column sums of all rows against integer numpy."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from eii import lib as L
from eii import synth


def _gemm(A, W):
    lib = L.load()
    M, K = A.shape
    N = W.shape[0]
    acc = torch.empty((M, N), dtype=torch.int64, device="cuda")
    At, Wt = torch.from_numpy(A).cuda(), torch.from_numpy(W).cuda()
    L.check(lib.eii_gemm_i8(At.data_ptr(), 16 if A.dtype == np.int16 else 32, Wt.data_ptr(), M, N, K,
                            acc.data_ptr(), None))
    torch.cuda.synchronize()
    return acc


@pytest.mark.parametrize("a_bits", [32, 16])
@pytest.mark.parametrize("K,N", synth.GEMM_SHAPES)
def test_gemm_sweep_exact(K, N, a_bits):
    A, W = synth.gemm_inputs(K, N, a_bits)
    print(f"K={K} N={N} a_bits={a_bits}", flush=True)
    acc = _gemm(A, W)
    Wd = W.astype(np.float64)
    if N <= 1536:
        want = np.rint(A.astype(np.float64) @ Wd.T).astype(np.int64)
        np.testing.assert_array_equal(acc.cpu().numpy(), want)
        return
    rows = np.unique(np.concatenate([[0, synth.GEMM_M - 1],
                                     np.random.default_rng(K + N + a_bits).integers(0, synth.GEMM_M, 510)]))
    got = acc[torch.from_numpy(rows).cuda()].cpu().numpy()
    np.testing.assert_array_equal(got, np.rint(A[rows].astype(np.float64) @ Wd.T).astype(np.int64))
    # sum over all rows: (sum_m A[m]) . W[n], exact in int64 (|sum| < 2^43 * 127 * 576 < 2^63)
    colsum = acc.sum(dim=0).cpu().numpy()
    np.testing.assert_array_equal(colsum, A.astype(np.int64).sum(axis=0) @ W.astype(np.int64).T)
