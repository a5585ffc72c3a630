"""Drop-in for python/intref.py backed by libeii on an MI355X.

    sys.path.insert(0, "<repo>/exact-integer-inference_amd"); import intref
    M = intref.Model(model_bin="model.bin")        # the file python/export_vectors.py writes
    logits = M.forward(ids)                         # int64 [T, 49152], f = 16, bit-exact

Same names, argument meanings and return types as python/intref.py (numpy int64 arrays in
and out, AssertionError on violated bounds, ValueError for a request outside what the engine
implements).  Differences, all deliberate:
  * Model takes the weights from a model.bin instead of the safetensors checkpoint
    (python/intref.py:132-151 quantizes those on load; model.bin is what that quantization
    produces, python/export_vectors.py:24-45); `wide=False` (the comparison mode whose
    formats model.bin does not record) raises.
  * forward/embed/block/rmsnorm/linear/matmul_exact run on the GPU through libeii.so and
    raise when it is missing; there is no CPU path.  rs, sat, dequant and the quantizers are
    the reference's host-side elementwise helpers (its callers apply them to host arrays).
  * block(..., trace) fills every key the reference's does (python/intref.py:183,198-285):
    resid_in/_mid/_out, _f, norm1/norm2 _U/_z/_out, the projections, q/k_rope, attn_score and
    attn_prob [9, T, T], attn_ctx, o_res, silu_gate, mlp_gated, down_res -- all computed on the
    GPU (the scores and probabilities by a trace-only kernel, o_res/down_res from the exact int64
    accumulators).
  * prop holds, for every format site the forward reads ("site|l", "final_out|30"), the class
    and k the reference's scaling_proposal.json entry implies, rebuilt from model.bin's fm
    records (flagged iff 32 bits; k = bits - 1 - f), as python/export_vectors.py:27,54 reads it.
  * forward_batch(ids [B, T]) is an addition: B independent sequences in one call.
"""
import math
import os

import numpy as np

from eii import modelbin as _mb
from eii import tables as _tables

F_RES = 15                        # python/intref.py:33-38
F_SCORE = 7
DMAX = 12 * 128
EXP_BITS = 30
EPS_S = 6184753
R_ISQRT = 40
I64 = np.int64


def rs(x, n):                     # python/intref.py:42-50
    if np.isscalar(n):
        n = int(n)
        if n <= 0:
            return x << (-n)
        return (x + (I64(1) << (n - 1))) >> n
    n = np.asarray(n, dtype=I64)
    assert (n >= 1).all(), "per-element shift must be >= 1"
    return (x + (I64(1) << (n - 1))) >> n


def sat(x, bits):                 # python/intref.py:53-55
    lo, hi = -(1 << (bits - 1)), (1 << (bits - 1)) - 1
    return np.clip(x, lo, hi)


from eii.quant import dequant   # noqa: E402  python/intref.py:311


def exp_table():                  # python/intref.py:72-77
    return _tables.exp_table()


def silu_table(f_in, f_out, out_bits):   # python/intref.py:80-93
    return _tables.silu_table(f_in, f_out, out_bits)


def rope_tables(T, theta=100000, head_dim=64):   # python/intref.py:96-108
    if theta != 100000 or head_dim != 64:
        raise ValueError("the engine's RoPE is theta = 100000, head_dim = 64")
    return _tables.rope_tables(T)


# quant_rows (python/intref.py:113-124), quant_vec_int16 (:127-130): eii/quant.py
from eii.quant import quant_rows, quant_vec_int16   # noqa: E402


# ---------------------------------------------------------------- GPU operators

def _torch():
    import torch
    if not torch.cuda.is_available():
        from eii.lib import EIIError, EII_E_DEVICE
        raise EIIError(EII_E_DEVICE, "intref: no GPU visible; this implementation runs only on the GPU")
    return torch


def _width(bound):
    if bound <= 1 << 7:
        return 8
    if bound <= 1 << 15:
        return 16
    if bound <= 1 << 31:
        return 32
    raise ValueError(f"activation bound {bound} exceeds the engine's 32-bit limb inputs")


_NP_OF_BITS = {8: np.int8, 16: np.int16, 32: np.int32}


def _fits(a, bits):
    a = np.asarray(a)
    return a.size == 0 or (int(a.min()) >= -(1 << (bits - 1)) and int(a.max()) < (1 << (bits - 1)))


def _dev(a, dtype):
    torch = _torch()
    return torch.from_numpy(np.array(a, dtype=dtype, order="C")).cuda()


def matmul_exact(A, Wf, bound_a, wmax=127):      # python/intref.py:58-63
    """Exact int64 A [T, K] @ W [N, K]^T on the int8 MFMA path (int8-valued W, |A| <= 2^31, any K)."""
    import ctypes as C
    from eii import lib as L
    A = np.asarray(A)
    K = A.shape[1]
    assert bound_a * wmax * K < 2.0 ** 53, "float64 accumulation would not be exact"
    W = np.asarray(Wf, dtype=np.float64)
    if W.min(initial=0) < -128 or W.max(initial=0) > 127 or np.any(W != np.rint(W)):
        raise ValueError("matmul_exact on the engine needs int8 weights")
    bits = _width(bound_a)
    if not _fits(A, bits):
        raise ValueError(f"A holds values outside the {bits}-bit range its bound {bound_a} implies")
    torch = _torch()
    a = _dev(A, _NP_OF_BITS[bits])
    w = _dev(W, np.int8)
    N = W.shape[0]
    pad = (-N) % 4                                   # the kernels take N in multiples of 4
    if pad:
        w = torch.cat([w, torch.zeros((pad, K), dtype=torch.int8, device=w.device)])
    acc = torch.empty((A.shape[0], N + pad), dtype=torch.int64, device=w.device)
    L.check(L.load().eii_gemm_i8(C.c_void_p(a.data_ptr()), bits, C.c_void_p(w.data_ptr()), A.shape[0], N + pad, K,
                                 C.c_void_p(acc.data_ptr()), C.c_void_p(torch.cuda.current_stream().cuda_stream)))
    return acc[:, :N].cpu().numpy()


class Model:
    """python/intref.py:132-301 over a model.bin held on one GPU."""

    def __init__(self, wide=True, proposal_path=None, model_bin=None, device=0):
        if not wide:
            raise ValueError("narrow comparison mode is not recorded in model.bin")
        path = model_bin or os.environ.get("EII_MODEL_BIN")
        if not path:
            raise ValueError("Model needs model_bin= (or EII_MODEL_BIN): the engine loads a model.bin")
        from eii.engine import Engine
        self.engine = Engine(path, device=device)
        self.bin = _mb.read(path)
        self.L = _mb.NL
        self.wide = True
        self.emb_q, self.emb_m, self.emb_n = self.bin.emb_q, self.bin.emb_m, self.bin.emb_n
        self.final_gain = self.bin.final_gain
        self.layers = [{k: L[k] for k in ("q", "k", "v", "o", "gate", "up", "down", "ln1", "ln2")}
                       for L in self.bin.layers]
        self.rope = (self.bin.rope_cos, self.bin.rope_sin)
        self.f_y = self.bin.f_y
        self.prop = self._prop()

    def _prop(self):
        """python/intref.py:138 `prop` for the sites the forward reads, rebuilt from the fm records:
        Model.fmt's rule (flagged -> (32, 31 - k), else (16, 15 - k)) inverted."""
        prop = {}
        for l in range(self.L):
            for site in _mb.SITES:
                bits, f = self.bin.fmt(site, l)
                prop[f"{site}|{l}"] = {"class": "flagged_wide_int32" if bits == 32 else "int16_per_tensor",
                                       "k": bits - 1 - f, "f": f}
        prop[f"final_out|{self.L}"] = {"class": "int16_per_tensor", "k": 15 - self.f_y, "f": self.f_y}
        return prop

    def fmt(self, site, l):                          # python/intref.py:154-160
        if site == "final_out" and l == self.L:
            return 16, self.f_y
        return self.bin.fmt(site, l)

    def embed(self, ids):                            # python/intref.py:163-166
        return self.engine.embed(np.asarray(ids, dtype=I64)).cpu().numpy().astype(I64)

    def rmsnorm(self, x, gain, f_out, bits_out, trace=None, tag=""):   # python/intref.py:168-184
        import ctypes as C
        from eii import lib as L
        torch = _torch()
        x = np.asarray(x)
        assert x.shape[1] == _mb.D and x.min(initial=0) >= -2 ** 31 and x.max(initial=0) < 2 ** 31
        wq, fw = gain
        if not _fits(wq, 32):
            raise ValueError("rmsnorm on the engine takes gains inside int32")
        xd, gd = _dev(x, np.int32), _dev(wq, np.int32)
        out = torch.empty(x.shape, dtype=torch.int16 if bits_out == 16 else torch.int32, device=xd.device)
        L.check(L.load().eii_rmsnorm(C.c_void_p(xd.data_ptr()), x.shape[0], C.c_void_p(gd.data_ptr()), fw, f_out,
                                     bits_out, C.c_void_p(out.data_ptr()),
                                     C.c_void_p(torch.cuda.current_stream().cuda_stream)))
        out = out.cpu().numpy().astype(I64)
        if trace is not None:
            trace[tag + "_out"] = out
        return out

    def linear(self, a, bound_a, W, f_in, f_out, bits_out):      # python/intref.py:186-190
        import ctypes as C
        from eii import lib as L
        torch = _torch()
        q, m, n = W
        acc = matmul_exact(a, q, bound_a)
        assert np.abs(acc).max() * int(m.max()) < 2 ** 63
        bits = _width(bound_a)
        a_d = _dev(a, _NP_OF_BITS[bits])
        w_d = _dev(q, np.int8)
        N, K = w_d.shape
        if N % 4:
            raise ValueError("linear on the engine needs N a multiple of 4")
        shift = np.asarray(n, dtype=I64) + f_in - f_out
        assert (shift >= 1).all(), "per-element shift must be >= 1"
        if not _fits(m, 32) or not _fits(shift, 32):
            raise ValueError("linear on the engine takes multipliers and shifts inside int32")
        ws = torch.empty(N, dtype=torch.int32, device=w_d.device)
        st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
        lib = L.load()
        L.check(lib.eii_weight_colsum(C.c_void_p(w_d.data_ptr()), N, K, C.c_void_p(ws.data_ptr()), st))
        m_d, s_d = _dev(m, np.int32), _dev(shift, np.int32)
        out = torch.empty((a_d.shape[0], N), dtype=torch.int16 if bits_out == 16 else torch.int32, device=w_d.device)
        L.check(lib.eii_linear(C.c_void_p(a_d.data_ptr()), bits, C.c_void_p(w_d.data_ptr()), C.c_void_p(ws.data_ptr()),
                               C.c_void_p(m_d.data_ptr()), C.c_void_p(s_d.data_ptr()), a_d.shape[0], N, K, bits_out,
                               C.c_void_p(out.data_ptr()), st))
        return out.cpu().numpy().astype(I64), acc

    def block(self, l, x, trace=None):               # python/intref.py:192-286
        torch = _torch()
        x = np.asarray(x)
        T = x.shape[0]
        xd = _dev(x, np.int32)
        if trace is not None:
            trace["resid_in"] = x.copy()
        bufs = self.engine.block(l, xd, 1, T, trace=trace is not None)
        out = xd.cpu().numpy().astype(I64)
        if trace is not None:
            for k, v in bufs.items():
                v = v.cpu().numpy().astype(I64)
                trace[k] = v[0] if k in ("attn_score", "attn_prob") else v   # [9, T, T] for the one sequence
            trace["resid_out"] = out.copy()
            f = {s: self.fmt(s, l)[1] for s in _mb.SITES}
            bits_m, f_m0 = self.fmt("mlp_gated", l)
            f["mlp_gated"] = min(f_m0, f["silu_gate"] + f["up_proj"]) if bits_m == 32 else f_m0
            trace["_f"] = {"resid_in": F_RES, "o_res": F_RES, "resid_mid": F_RES, "down_res": F_RES,
                           "resid_out": F_RES, "attn_score": F_SCORE, "attn_prob": 16, **f}
        return out

    def forward(self, ids, narrow_residual=False):   # python/intref.py:288-301
        if narrow_residual:
            raise ValueError("narrow_residual is an ablation mode outside the engine")
        ids = np.asarray(ids, dtype=I64).reshape(-1)
        return self.forward_batch(ids[None, :])[0]

    def forward_batch(self, ids):
        """ids int64 [B, T] -> logits int64 [B, T, 49152]: B independent sequences."""
        out = self.engine.forward(np.asarray(ids, dtype=I64), logits=True)
        return out["logits"].cpu().numpy().astype(I64)
