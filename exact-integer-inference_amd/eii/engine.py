"""GPU engine: a loaded model.bin on one MI355X, driven through libeii's C ABI.

torch provides device memory and the current HIP stream; all arithmetic runs in the
library's gfx950 kernels.  Tensors passed in must live on the engine's device.
"""
import ctypes as C

import numpy as np
import torch

from . import lib as L
from . import modelbin as mb
from .tables import rope_tables

V, D, NL = mb.V, mb.D, mb.NL


def _ptr(t):
    return C.c_void_p(t.data_ptr()) if t is not None else None


def _stream():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


class Engine:
    """A model.bin resident on `device` (python/intref.py Model, batched and on the GPU)."""

    def __init__(self, model_bin, device=0, rope_rows=None):
        if not torch.cuda.is_available():
            raise L.EIIError(L.EII_E_DEVICE, "no GPU visible to torch")
        self.lib = L.load()
        self.device = torch.device("cuda", device)
        torch.cuda.set_device(self.device)
        h = C.c_void_p()
        L.check(self.lib.eii_model_load(str(model_bin).encode(), device, C.byref(h)))
        self.h = h
        self.path = str(model_bin)
        if rope_rows and rope_rows > mb.ROPE_POS:
            self.set_rope(rope_rows)

    def close(self):
        if getattr(self, "h", None):
            self.lib.eii_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ------------------------------------------------------------------ model data
    def set_rope(self, rows):
        """Load RoPE tables for positions 0..rows-1 (python/intref.py:96-108)."""
        Ct, St = rope_tables(rows)
        Ct = np.ascontiguousarray(Ct, dtype=np.int64)
        St = np.ascontiguousarray(St, dtype=np.int64)
        L.check(self.lib.eii_model_set_rope(self.h, Ct.ctypes.data_as(L.i64p), St.ctypes.data_as(L.i64p), rows))

    @property
    def rope_rows(self):
        return self.lib.eii_model_rope_rows(self.h)

    def formats(self, layer):
        fm = np.zeros(24, dtype=np.int64)
        fy = np.zeros(1, dtype=np.int64)
        L.check(self.lib.eii_model_formats(self.h, layer, fm.ctypes.data_as(L.i64p), fy.ctypes.data_as(L.i64p)))
        return fm, int(fy[0])

    def set_graphs(self, on=True):
        """Replay whole forwards as HIP graphs (captured per batch shape and output buffers)."""
        L.check(self.lib.eii_model_set_graphs(self.h, 1 if on else 0))

    def ensure_rope(self, T):
        if T > self.rope_rows:
            self.set_rope(max(T, 2 * self.rope_rows))

    # ------------------------------------------------------------------ forward
    def forward(self, ids, embed=False, resid=False, logits=True, check=True, dump=None):
        """ids int64 [B, T] (torch on the device, or numpy) -> dict of device tensors:
        'embed' int32 [S, T, 576], 'resid' int32 [30, S, T, 576], 'logits' int32 [B, T, 49152],
        where the S dumped sequences are the indices in `dump` (in batch order; None = all B)."""
        ids = self._ids(ids)
        B, T = ids.shape
        self.ensure_rope(T)
        mask = _dump_mask(B, dump)
        S = B if mask is None else int(mask.sum())
        out = self._alloc(S * T, embed, resid, False)
        if logits:
            out["logits"] = torch.empty((B * T, V), dtype=torch.int32, device=self.device)
        L.check(self.lib.eii_forward(self.h, _ptr(ids), B, T, _ptr(out.get("embed")), _ptr(out.get("resid")),
                                     _ptr(out.get("logits")), _mask_ptr(mask), _stream()))
        if check:
            self.check()
        r = {k: (v.view(NL, S, T, -1) if k == "resid" else v.view(S, T, -1)) for k, v in out.items() if k != "logits"}
        if logits:
            r["logits"] = out["logits"].view(B, T, -1)
        return r

    def forward_packed(self, ids, seq_lens, embed=False, resid=False, logits=True, check=True, dump=None):
        """Ragged batch: ids int64 [sum(seq_lens)] packed sequence after sequence; 'embed' and
        'resid' hold the rows of the sequences in `dump` (None = all), packed."""
        ids = self._ids(ids).reshape(-1)
        lens = np.ascontiguousarray(seq_lens, dtype=np.int32)
        assert int(lens.sum()) == ids.numel()
        self.ensure_rope(int(lens.max()))
        mask = _dump_mask(len(lens), dump)
        rows = ids.numel() if mask is None else int(lens[mask.astype(bool)].sum())
        out = self._alloc(rows, embed, resid, False)
        if logits:
            out["logits"] = torch.empty((ids.numel(), V), dtype=torch.int32, device=self.device)
        L.check(self.lib.eii_forward_packed(self.h, _ptr(ids), lens.ctypes.data_as(L.i32p), len(lens),
                                            _ptr(out.get("embed")), _ptr(out.get("resid")),
                                            _ptr(out.get("logits")), _mask_ptr(mask), _stream()))
        if check:
            self.check()
        return out

    def check(self):
        L.check(self.lib.eii_check(self.h, _stream()))

    def block(self, layer, x, B, T, trace=False):
        """x int32 [B*T, 576] device tensor, updated in place; returns the trace dict if asked."""
        self.ensure_rope(T)
        tr = None
        bufs = {}
        if trace:
            fm, _ = self.formats(layer)
            bits = {s: int(fm[2 * i]) for i, s in enumerate(mb.SITES)}
            width = {"norm1_out": D, "q_proj": D, "k_proj": 192, "v_proj": 192, "q_rope": D, "k_rope": 192,
                     "attn_ctx": D, "norm2_out": D, "gate_proj": 1536, "up_proj": 1536, "mlp_gated": 1536}
            for s, w in width.items():
                dt = torch.int16 if bits[s] == 16 else torch.int32
                bufs[s] = torch.empty((B * T, w), dtype=dt, device=self.device)
            dev, M = self.device, B * T
            bufs["resid_mid"] = torch.empty((M, D), dtype=torch.int32, device=dev)
            # norm internals, attention matrices and the unsaturated residual updates (include/eii.h)
            for n in ("norm1", "norm2"):
                bufs[n + "_U"] = torch.empty(M, dtype=torch.int32, device=dev)
                bufs[n + "_z"] = torch.empty((M, D), dtype=torch.int32, device=dev)
            bufs["attn_score"] = torch.empty((B, 9, T, T), dtype=torch.int16, device=dev)
            bufs["attn_prob"] = torch.empty((B, 9, T, T), dtype=torch.int32, device=dev)
            bufs["o_res"] = torch.empty((M, D), dtype=torch.int64, device=dev)
            bufs["down_res"] = torch.empty((M, D), dtype=torch.int64, device=dev)
            bufs["silu_gate"] = torch.empty((M, 1536), dtype=torch.int32, device=dev)
            tr = L.eii_trace(**{k: v.data_ptr() for k, v in bufs.items()})
        L.check(self.lib.eii_block(self.h, layer, _ptr(x), B, T, C.byref(tr) if tr is not None else None, _stream()))
        return bufs

    def embed(self, ids):
        ids = self._ids(ids).reshape(-1)
        x = torch.empty((ids.numel(), D), dtype=torch.int32, device=self.device)
        L.check(self.lib.eii_embed(self.h, _ptr(ids), ids.numel(), _ptr(x), _stream()))
        self.check()
        return x

    def final(self, x):
        M = x.shape[0]
        lg = torch.empty((M, V), dtype=torch.int32, device=self.device)
        L.check(self.lib.eii_final(self.h, _ptr(x), M, _ptr(lg), _stream()))
        self.check()
        return lg

    # ------------------------------------------------------------------ decoding
    def kv_cache(self, B, max_T):
        """A KV cache for incremental decoding of B sequences of up to max_T positions."""
        return KVCache(self, B, max_T)

    def argmax(self, logits):
        """int64 [rows]: the lowest index of each row's largest logit (numpy.argmax's tie rule)."""
        lg = logits.reshape(-1, logits.shape[-1]).contiguous()
        out = torch.empty(lg.shape[0], dtype=torch.int64, device=self.device)
        L.check(self.lib.eii_argmax(_ptr(lg), lg.shape[0], lg.shape[1], _ptr(out), _stream()))
        return out

    def generate(self, prompt, n):
        """Greedy continuation of n tokens after prompt int64 [B, T0] with a KV cache; returns
        (tokens int64 [B, n], logits of every position int32 [B, T0 + n - 1, 49152] on the device)."""
        prompt = self._ids(prompt)
        B, T0 = prompt.shape
        self.ensure_rope(T0 + n)
        kv = self.kv_cache(B, T0 + n)
        try:
            logits = [kv.append(prompt)]
            toks = [self.argmax(logits[-1][:, -1])]
            for _ in range(n - 1):
                logits.append(kv.append(toks[-1][:, None]))
                toks.append(self.argmax(logits[-1][:, -1]))
        finally:
            kv.close()
        return torch.stack(toks, dim=1), torch.cat(logits, dim=1)

    # ------------------------------------------------------------------ helpers
    def _ids(self, ids):
        if isinstance(ids, np.ndarray):
            ids = torch.from_numpy(np.ascontiguousarray(ids, dtype=np.int64))
        ids = ids.to(device=self.device, dtype=torch.int64).contiguous()
        if ids.dim() == 1:
            ids = ids[None, :]
        return ids

    def _alloc(self, M, embed, resid, logits):
        out = {}
        if embed:
            out["embed"] = torch.empty((M, D), dtype=torch.int32, device=self.device)
        if resid:
            out["resid"] = torch.empty((NL, M, D), dtype=torch.int32, device=self.device)
        if logits:
            out["logits"] = torch.empty((M, V), dtype=torch.int32, device=self.device)
        return out

    @staticmethod
    def _shape(out, bt):
        B, T = bt
        r = {}
        for k, v in out.items():
            r[k] = v.view(NL, B, T, -1) if k == "resid" else v.view(B, T, -1)
        return r


def _dump_mask(n, dump):
    """uint8 [n] with 1 at the sequence indices in dump, or None for every sequence."""
    if dump is None:
        return None
    mask = np.zeros(n, dtype=np.uint8)
    idx = np.asarray(dump, dtype=np.int64)
    assert idx.size == 0 or (idx.min() >= 0 and idx.max() < n), "dump indices outside the batch"
    mask[idx] = 1
    return mask


def _mask_ptr(mask):
    return None if mask is None else mask.ctypes.data_as(C.c_void_p)


class KVCache:
    """Incremental decoding state on an Engine's device: per layer the q|k|v rows and V^T planes of
    every position appended so far, for B sequences of up to max_T positions.

    No counterpart in python/intref.py, whose forward recomputes every position over the full
    prefix; the cache is the reference's stated next step (exact-integer-inference.tex:167).  Each
    position depends only on its prefix, so appended positions get the logits a full forward over
    the whole sequence gives them.
    """

    def __init__(self, engine, B, max_T):
        self.engine = engine
        self.B = B
        engine.ensure_rope(max_T)
        h = C.c_void_p()
        L.check(engine.lib.eii_kv_create(engine.h, B, max_T, C.byref(h)))
        self.h = h

    @property
    def length(self):
        return self.engine.lib.eii_kv_length(self.h)

    def reset(self):
        L.check(self.engine.lib.eii_kv_reset(self.h))

    def append(self, ids, logits=True, check=True):
        """ids int64 [B, T_new] -> logits int32 [B, T_new, 49152] of the new positions (or None)."""
        e = self.engine
        ids = e._ids(ids)
        if ids.shape[0] != self.B:
            raise L.EIIError(L.EII_E_ARG, f"expected {self.B} sequences, got {ids.shape[0]}")
        T_new = ids.shape[1]
        lg = torch.empty((self.B, T_new, V), dtype=torch.int32, device=e.device) if logits else None
        L.check(e.lib.eii_kv_append(e.h, self.h, _ptr(ids), T_new, _ptr(lg), _stream()))
        if check:
            e.check()
        return lg

    def close(self):
        if getattr(self, "h", None):
            self.engine.lib.eii_kv_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
