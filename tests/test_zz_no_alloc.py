"""eii_gemm_i8_ws_noalloc (the allocation-free exact matmul) against eii_gemm_i8_ws through the C ABI:
two calls in a row, the second smaller, each bit-equal to the allocating entry point; sizes past the
fixed scratch are a bound error before any device work."""
import ctypes as C

import numpy as np
import pytest
import torch

from eii import lib as L

pytestmark = pytest.mark.gpu


def _call(fn, A, a_bits, W, ws, acc):
    M, K = A.shape
    N = W.shape[0]
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    return fn(C.c_void_p(A.data_ptr()), a_bits, C.c_void_p(W.data_ptr()), C.c_void_p(ws.data_ptr()), M, N, K,
              C.c_void_p(acc.data_ptr()), stream)


def test_noalloc_matches_allocating_entry():
    lib = L.load()
    rng = np.random.default_rng(21)
    dt = {8: np.int8, 16: np.int16, 32: np.int32}
    # (a_bits, M, N, K): the second call of each pair is smaller and leaves stale bytes of the first
    for a_bits, shapes in ((32, ((4096, 576, 1536), (300, 192, 576))), (16, ((2048, 1536, 576), (37, 64, 100))),
                           (8, ((512, 576, 577), (5, 4, 64)))):
        for M, N, K in shapes:
            lo, hi = -(1 << (a_bits - 1)), 1 << (a_bits - 1)
            A = rng.integers(lo, hi, size=(M, K)).astype(dt[a_bits])
            A.flat[0], A.flat[-1] = lo, hi - 1
            W = rng.integers(-128, 128, size=(N, K)).astype(np.int8)
            At, Wt = torch.from_numpy(A).cuda(), torch.from_numpy(W).cuda()
            ws = torch.empty(N, dtype=torch.int32, device="cuda")
            L.check(lib.eii_weight_colsum(C.c_void_p(Wt.data_ptr()), N, K, C.c_void_p(ws.data_ptr()),
                                          C.c_void_p(torch.cuda.current_stream().cuda_stream)))
            want = torch.empty((M, N), dtype=torch.int64, device="cuda")
            got = torch.full((M, N), -1, dtype=torch.int64, device="cuda")
            L.check(_call(lib.eii_gemm_i8_ws, At, a_bits, Wt, ws, want))
            L.check(_call(lib.eii_gemm_i8_ws_noalloc, At, a_bits, Wt, ws, got))
            torch.cuda.synchronize()
            assert torch.equal(got, want), (a_bits, M, N, K)
            if M * N <= 1 << 16:
                ref = (A.astype(object) @ W.astype(object).T).astype(np.int64)
                assert np.array_equal(got.cpu().numpy(), ref), (a_bits, M, N, K)


def test_noalloc_rejects_oversize():
    lib = L.load()
    A = torch.zeros((1 << 15, 1024), dtype=torch.int32, device="cuda")   # 128 MiB of limb planes
    W = torch.zeros((64, 1024), dtype=torch.int8, device="cuda")
    ws = torch.zeros(64, dtype=torch.int32, device="cuda")
    acc = torch.empty((1 << 15, 64), dtype=torch.int64, device="cuda")
    assert _call(lib.eii_gemm_i8_ws_noalloc, A, 32, W, ws, acc) == L.EII_E_BOUND
    assert b"64 MiB" in lib.eii_last_error()
