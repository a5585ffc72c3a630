"""CPU model of the GEMM and attention kernels' index maps (csrc/index_maps.h, the functions the
kernels compute their addresses with), in the spirit of the reference's CPU emulation of its CUDA
kernels (cuda/emulate/make_emu.py:4-35, cuda/emulate/shim.h:46-63).

For every tile shape the kernels instantiate, the model runs a whole launch on the CPU: the
direct-to-LDS activation loads into a simulated stage (through the LDS swizzle), the fragment reads,
v_mfma_i32_32x32x32_i8 from its documented operand and result layouts, the skinny shapes' K split and
partial-sum reduction, and the epilogue's element map.  It checks every limb sum against a direct
sum, every global and LDS access against its buffer, that no LDS slot is written twice or read
unwritten, and that every output element is stored exactly once.  Planted index mistakes (in the
model, on the CPU) must be caught."""
import ctypes as C

import numpy as np
import pytest

from eii import lib as L

SQUARE, NARROW, ROW, SKINNY, SKINNY32 = 0, 1, 2, 3, 4


@pytest.fixture(scope="module")
def hc():
    return L.load_hostcheck()


def run(hc, aw, shape, M, N, K, a_kb=64, seed=1, plant=0):
    st = np.zeros(6, dtype=np.int64)
    err = hc.eii_host_gemm_model(aw, shape, M, N, K, a_kb, seed, plant, C.c_void_p(st.ctypes.data))
    return err, st


# (limbs, shape, M, N, K, K-block width): every shape the kernels launch, with ragged M and N, both
# plane layouts, and the model's K depths 576 and 1536 at the smallest M that still shows the maps
CASES = [
    (2, SQUARE, 200, 256, 128, 64),
    (4, SQUARE, 100, 200, 128, 64),
    (4, SQUARE, 70, 576, 192, 32),      # down projection: gated planes in 32-byte K blocks
    (2, NARROW, 130, 576, 128, 64),
    (2, ROW, 100, 960, 128, 64),        # q/k/v: the last column tile a quarter full
    (2, ROW, 65, 3072, 64, 64),
    (2, SKINNY, 1, 3072, 576, 64),      # decoding: gate/up
    (2, SKINNY, 17, 960, 576, 64),
    (2, SKINNY, 200, 3072, 128, 64),   # skinny tiles serve up to 256 rows
    (4, SKINNY32, 129, 576, 192, 32),
    (4, SKINNY32, 3, 576, 1536, 32),    # decoding: down
    (2, SKINNY32, 32, 576, 576, 64),
    (4, SKINNY, 5, 128, 192, 64),
]


@pytest.mark.parametrize("aw,shape,M,N,K,a_kb", CASES)
def test_gemm_index_maps(hc, aw, shape, M, N, K, a_kb):
    err, st = run(hc, aw, shape, M, N, K, a_kb)
    assert err == 0, f"wrong sums {st[1]}, out of bounds {st[2]}, LDS slots {st[3]}, stores {st[4]}"
    assert st[5] == aw * M * N          # every output element's limb sums compared once


@pytest.mark.parametrize("plant,aw,shape,M,N,K,what", [
    (1, 2, ROW, 64, 256, 64, 1),        # fragment reads without the LDS swizzle: wrong sums
    (2, 2, SQUARE, 128, 128, 64, 1),    # result rows off by a row group: wrong sums
    (3, 4, SKINNY32, 1, 64, 1536, 1),   # skinny K split loses a slice: wrong sums
])
def test_gemm_model_catches_planted_mistakes(hc, plant, aw, shape, M, N, K, what):
    err, st = run(hc, aw, shape, M, N, K, plant=plant)
    assert err > 0 and st[what] > 0


def test_gemm_model_rejects_unknown_shapes(hc):
    assert run(hc, 4, ROW, 64, 256, 64)[0] == -1      # row tiles exist for 2-limb inputs only
    assert run(hc, 2, SQUARE, 64, 128, 100)[0] == -1  # K not a multiple of 64


def test_attention_layouts(hc):
    assert hc.eii_host_attn_model(7, 0) == 0
    assert hc.eii_host_attn_model(7, 1) > 0           # planted: key order without the row-group swap


def test_attention_score_digits(hc):
    # every int16 query and key element, and 4000 random and extreme 64-dimension rows
    assert hc.eii_host_attn_digits(11, 0) == 0
    assert hc.eii_host_attn_digits(11, 1) > 0         # planted: the extra 0/1 digit of q >= 32640 dropped


def _dist_table_index(rm, sp, hi_bound=True):
    # kernels.hip attn_kernel scores(), MODE Dist, score shift >= 16: s' = wv >> (sh - 16) and the
    # exp table index as one median of three
    hi = np.minimum(1537, rm + 32768) if hi_bound else np.full_like(rm, 1537)
    return np.clip(rm - sp, rm - 32767, hi)


def test_attention_table_index_median():
    # the index the exp lookups use, min(rowmax - SAT16(s'), 1537) (python/intref.py:239-244, with
    # index 1537 holding 0), for every shifted score s' of the int32 range the kernels form and
    # every row max that is the max of its row's saturated scores (rm >= SAT16(s'))
    rng = np.random.default_rng(16)
    sp = np.concatenate([rng.integers(-2**31, 2**31, 400000), np.arange(-34000, 34000),
                         [-2**31, 2**31 - 1, -32769, -32768, 32767, 32768]]).astype(np.int64)
    rm = np.concatenate([rng.integers(-32768, 32768, sp.size - 8), [-32768, -32768, -31232, -31231, 32767, 32767,
                                                                     0, -1]]).astype(np.int64)
    sat = np.clip(sp, -32768, 32767)
    rm = np.maximum(rm, sat)   # a row max is at least every score of its row
    want = np.minimum(rm - sat, 1537)
    assert np.array_equal(_dist_table_index(rm, sp), want)
    # every row max from -32768 upward against the scores that saturate low and high
    rm2 = np.arange(-32768, 32768, dtype=np.int64)
    for s in (-2**31, -40000, -32769, -32768):
        assert np.array_equal(_dist_table_index(rm2, np.full_like(rm2, s)), np.minimum(rm2 + 32768, 1537))
    assert np.array_equal(_dist_table_index(np.array([32767]), np.array([2**31 - 1])), np.array([0]))
    # planted: the upper bound without rm + 32768 (rows whose max lies within 1536 of -32768)
    assert not np.array_equal(_dist_table_index(rm2, np.full_like(rm2, -40000), hi_bound=False),
                              np.minimum(rm2 + 32768, 1537))


@pytest.mark.parametrize("N,K", [(576, 576), (960, 576), (100, 64), (33, 1536)])
def test_weight_fragment_order(hc, N, K):
    assert hc.eii_host_wfrag_model(N, K) == 0
