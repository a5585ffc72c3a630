"""ORACLE (test infrastructure only): numpy restatement of python/intref.py.

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg import this module,
and only to check the HIP engine's results; the engine never calls it.

It restates the integer semantics of python/intref.py step by step (each function cites
the lines it follows) over a model.bin image read by its own reader (the layout of
python/export_vectors.py:24-45).  Matrix products go through float64 BLAS exactly as the
reference does (python/intref.py:58-63): every operand bound is asserted to keep all
partial sums below 2^53, so the products are exact integers.  Sequences of a batch are
independent: row-wise steps run on all rows at once, attention runs per sequence.

How it is pinned (tests/test_oracle.py): the reference's own scalar C program
(c/intref.c, built from /root/reference into oracle/_ref/) checks vectors this oracle
exports and must print ALL STATES EXACT; brute-force Python-int evaluation on tiny
shapes pins rs/sat/rmsnorm/linear/attention; closed-form properties pin the rest.
"""
import math
import os

import numpy as np

I64 = np.int64
V, D, DFF, NH, NKV, HD, NL = 49152, 576, 1536, 9, 3, 64, 30
F_RES, F_SCORE = 15, 7                    # python/intref.py:33-34
DMAX = 12 * 128                           # python/intref.py:35
EPS_S = 6184753                           # python/intref.py:37
R_ISQRT = 40                              # python/intref.py:38
ROPE_POS = 512
SITES = ("norm1_out", "q_proj", "k_proj", "v_proj", "q_rope", "k_rope", "attn_ctx",
         "norm2_out", "gate_proj", "up_proj", "silu_gate", "mlp_gated")
MATS = (("q", 576, 576), ("k", 192, 576), ("v", 192, 576), ("o", 576, 576),
        ("gate", 1536, 576), ("up", 1536, 576), ("down", 576, 1536))


def rs(x, n):                                        # python/intref.py:42-50
    if np.isscalar(n):
        n = int(n)
        if n <= 0:
            return x << (-n)
        return (x + (I64(1) << (n - 1))) >> n
    n = np.asarray(n, dtype=I64)
    assert (n >= 1).all(), "per-element shift must be >= 1"
    return (x + (I64(1) << (n - 1))) >> n


def sat(x, bits):                                    # python/intref.py:53-55
    lo, hi = -(1 << (bits - 1)), (1 << (bits - 1)) - 1
    return np.clip(x, lo, hi)


def matmul_exact(A, W, bound_a, wmax=127):           # python/intref.py:58-63
    """Exact int64 A[T,K] @ W[N,K]^T through float64 BLAS under the 2^53 bound."""
    K = A.shape[1]
    assert bound_a * wmax * K < 2.0 ** 53, "float64 accumulation would not be exact"
    out = np.asarray(A, dtype=np.float64) @ np.asarray(W, dtype=np.float64).T
    return np.rint(out).astype(I64)


def silu_gate(silu, g, u, f_s, f_u, f_m, bits_m):   # python/intref.py:272-276
    """SAT(RS(SILU[g + 32768] * u, f_s + f_u - f_m), bits_m), f_m already the reference's
    min(f_m0, f_s + f_u) for 32-bit gated values."""
    return sat(rs(silu[g + 32768] * u, f_s + f_u - f_m), bits_m)


class OracleModel:
    """A model.bin image read into int64 numpy arrays (c/intref.c:70-91 read order)."""

    def __init__(self, path, rope_rows=None):
        raw = np.fromfile(path, dtype=np.uint8)
        off = 0

        def take(dt, n):
            nonlocal off
            a = np.frombuffer(raw, dtype=dt, count=n, offset=off)
            off += a.nbytes
            return a

        i8, i64 = np.dtype(np.int8), np.dtype("<i8")
        self.emb_q = take(i8, V * D).reshape(V, D)
        self.emb_m = take(i64, V).astype(I64)
        self.emb_n = take(i64, V).astype(I64)
        self.fg_q = take(i64, D).astype(I64)
        self.fg_f = int(take(i64, 1)[0])
        self.f_y = int(take(i64, 1)[0])
        self.exp_tab = take(i64, DMAX + 1).astype(I64)
        self.rope_c = take(i64, ROPE_POS * 32).reshape(ROPE_POS, 32).astype(I64)
        self.rope_s = take(i64, ROPE_POS * 32).reshape(ROPE_POS, 32).astype(I64)
        self.layers = []
        for _ in range(NL):
            L = {"fm": [int(v) for v in take(i64, 24)]}
            L["ln1"] = (take(i64, D).astype(I64), int(take(i64, 1)[0]))
            L["ln2"] = (take(i64, D).astype(I64), int(take(i64, 1)[0]))
            for name, N, K in MATS:
                q = take(i8, N * K).reshape(N, K)
                L[name] = (q, take(i64, N).astype(I64), take(i64, N).astype(I64))
            L["silu"] = take(i64, 65536).astype(I64)
            self.layers.append(L)
        assert off == raw.size, "model.bin size does not match its layout"
        self._wf = {}

    def extend_rope(self, T):
        """RoPE rows beyond the 512 in model.bin, from the same closed form (python/intref.py:96-108)."""
        if T <= self.rope_c.shape[0]:
            return
        from .tables_ref import rope_tables
        C, S = rope_tables(T, start=self.rope_c.shape[0])
        self.rope_c = np.concatenate([self.rope_c, C])
        self.rope_s = np.concatenate([self.rope_s, S])

    def fmt(self, site, l):                          # python/intref.py:154-160 via the fm record
        i = SITES.index(site)
        fm = self.layers[l]["fm"]
        return fm[2 * i], fm[2 * i + 1]

    def wf(self, key, q):
        if key not in self._wf:
            self._wf[key] = np.asarray(q, dtype=np.float64)
        return self._wf[key]

    # ---------------------------------------------------------------- steps
    def embed(self, ids):                            # python/intref.py:163-166
        ids = np.asarray(ids).reshape(-1)
        q = self.emb_q[ids].astype(I64)
        x = q * self.emb_m[ids][:, None]
        return rs(x, (self.emb_n[ids] - F_RES)[:, None])

    def rmsnorm(self, x, gain, f_out, bits_out, trace=None, tag=""):   # python/intref.py:168-184
        T = x.shape[0]
        hi = x >> 16
        lo = x & 0xFFFF
        A = (hi * hi).sum(1); B = (hi * lo).sum(1); C = (lo * lo).sum(1)
        U = np.empty(T, dtype=I64)
        for t in range(T):
            S = (int(A[t]) << 32) + (int(B[t]) << 17) + int(C[t])
            U[t] = math.isqrt((1 << (2 * R_ISQRT)) // (S + EPS_S))
        z = rs(x * U[:, None], 16)
        wq, fw = gain
        acc = z * wq[None, :] * 3
        out = sat(rs(acc, 21 + fw - f_out), bits_out)
        if trace is not None:
            trace[tag + "_U"] = U; trace[tag + "_z"] = z; trace[tag + "_out"] = out
        return out

    def linear(self, a, bound_a, W, f_in, f_out, bits_out, key=None):   # python/intref.py:186-190
        q, m, n = W
        acc = matmul_exact(a, self.wf(key, q) if key else q, bound_a)
        assert np.abs(acc).max() * int(m.max()) < 2 ** 63
        return sat(rs(acc * m[None, :], n + f_in - f_out), bits_out), acc

    def rope(self, a, nheads, pos, f_in, f_o, bits_o):    # python/intref.py:212-222
        R = a.shape[0]
        a = a.reshape(R, nheads, HD)
        a1, a2 = a[:, :, :32], a[:, :, 32:]
        c, s = self.rope_c[pos][:, None, :], self.rope_s[pos][:, None, :]
        o1 = a1 * c - a2 * s
        o2 = a2 * c + a1 * s
        return sat(rs(np.concatenate([o1, o2], axis=2), 30 + f_in - f_o), bits_o)

    def attention(self, qr, kr, vv, shift_s, f_v, f_c, bits_c, bits_qr, bits_kr, bits_v,
                  trace=None):                        # python/intref.py:227-254
        """One sequence: qr [T, 9, 64], kr/vv [T, 3, 64] -> ctx [T, 9, 64]."""
        T = qr.shape[0]
        bq, bk, bv = 1 << (bits_qr - 1), 1 << (bits_kr - 1), 1 << (bits_v - 1)
        E = self.exp_tab
        ctx = np.empty((T, NH, HD), dtype=I64)
        causal = np.tril(np.ones((T, T), dtype=bool))
        for hh in range(NH):
            g = hh // 3
            acc = matmul_exact(qr[:, hh, :], kr[:, g, :], bq, wmax=bk)
            s = sat(rs(acc, shift_s), 16)
            rowmax = np.where(causal, s, -(1 << 40)).max(1, keepdims=True)
            d = rowmax - s
            valid = causal & (d <= DMAX)
            e = np.where(valid, E[np.clip(d, 0, DMAX)], 0)
            Z = e.sum(1, keepdims=True)
            P = (e * 65536 + Z // 2) // Z
            assert 65536 * bv * T < 2 ** 53
            acc2 = np.rint(P.astype(np.float64) @ vv[:, g, :].astype(np.float64)).astype(I64)
            ctx[:, hh, :] = sat(rs(acc2, 16 + f_v - f_c), bits_c)
            if trace is not None:
                trace.setdefault("attn_score", []).append(np.where(causal, s, 0))
                trace.setdefault("attn_prob", []).append(P)
        return ctx

    def block(self, l, x, seq_len, trace=None):       # python/intref.py:192-286
        """x int64 [B*seq_len, 576], B independent sequences of seq_len tokens each."""
        R = x.shape[0]
        T = seq_len
        B = R // T
        assert B * T == R
        Ly = self.layers[l]
        tr = trace
        self.extend_rope(T)
        pos = np.tile(np.arange(T), B)
        if tr is not None:
            tr["resid_in"] = x.copy()
            tr["_f"] = {"resid_in": F_RES, "o_res": F_RES, "resid_mid": F_RES, "down_res": F_RES,
                        "resid_out": F_RES, "attn_score": F_SCORE, "attn_prob": 16}   # python/intref.py:199-201

        bits_h, f_h = self.fmt("norm1_out", l)
        h = self.rmsnorm(x, Ly["ln1"], f_h, bits_h, tr, "norm1")
        bh = 1 << (bits_h - 1)
        bits_q, f_q = self.fmt("q_proj", l); bits_k, f_k = self.fmt("k_proj", l)
        bits_v, f_v = self.fmt("v_proj", l)
        q, _ = self.linear(h, bh, Ly["q"], f_h, f_q, bits_q, (l, "q"))
        k, _ = self.linear(h, bh, Ly["k"], f_h, f_k, bits_k, (l, "k"))
        v, _ = self.linear(h, bh, Ly["v"], f_h, f_v, bits_v, (l, "v"))
        bits_qr, f_qr = self.fmt("q_rope", l); bits_kr, f_kr = self.fmt("k_rope", l)
        qr = self.rope(q, NH, pos, f_q, f_qr, bits_qr)
        kr = self.rope(k, NKV, pos, f_k, f_kr, bits_kr)
        if tr is not None:
            tr.update(norm1_out=h, q_proj=q, k_proj=k, v_proj=v,
                      q_rope=qr.reshape(R, -1), k_rope=kr.reshape(R, -1))

        shift_s = f_qr + f_kr + 3 - F_SCORE
        assert shift_s >= 1
        bits_c, f_c = self.fmt("attn_ctx", l)
        vv = v.reshape(R, NKV, HD)
        ctx = np.empty((R, NH, HD), dtype=I64)
        if tr is not None and B == 1:
            tr["attn_score"], tr["attn_prob"] = [], []
        for b in range(B):
            sl = slice(b * T, (b + 1) * T)
            ctx[sl] = self.attention(qr[sl], kr[sl], vv[sl], shift_s, f_v, f_c, bits_c,
                                     bits_qr, bits_kr, bits_v, tr if B == 1 else None)
        ctx = ctx.reshape(R, D)
        if tr is not None:
            tr["attn_ctx"] = ctx
            if B == 1:                                            # python/intref.py:252-253
                tr["attn_score"] = np.stack(tr["attn_score"]); tr["attn_prob"] = np.stack(tr["attn_prob"])

        q_o, m_o, n_o = Ly["o"]                                   # python/intref.py:257-261
        acc = matmul_exact(ctx, self.wf((l, "o"), q_o), 1 << (bits_c - 1))
        assert np.abs(acc).max() * int(m_o.max()) < 2 ** 63
        o_res = rs(acc * m_o[None, :], n_o + f_c - F_RES)
        x = sat(x + o_res, 32)
        if tr is not None:
            tr["o_res"] = o_res; tr["resid_mid"] = x.copy()

        bits_h2, f_h2 = self.fmt("norm2_out", l)                  # python/intref.py:264-283
        h2 = self.rmsnorm(x, Ly["ln2"], f_h2, bits_h2, tr, "norm2")
        bh2 = 1 << (bits_h2 - 1)
        bits_g, f_g = self.fmt("gate_proj", l); bits_u, f_u = self.fmt("up_proj", l)
        g_, _ = self.linear(h2, bh2, Ly["gate"], f_h2, f_g, bits_g, (l, "gate"))
        u_, _ = self.linear(h2, bh2, Ly["up"], f_h2, f_u, bits_u, (l, "up"))
        bits_s, f_s = self.fmt("silu_gate", l)
        sg = Ly["silu"][g_ + 32768]
        bits_m, f_m0 = self.fmt("mlp_gated", l)
        f_m = min(f_m0, f_s + f_u) if bits_m == 32 else f_m0
        gated = silu_gate(Ly["silu"], g_, u_, f_s, f_u, f_m, bits_m)
        q_d, m_d, n_d = Ly["down"]
        acc = matmul_exact(gated, self.wf((l, "down"), q_d), 1 << (bits_m - 1))
        assert np.abs(acc).max() * int(m_d.max()) < 2 ** 63
        d_res = rs(acc * m_d[None, :], n_d + f_m - F_RES)
        x = sat(x + d_res, 32)
        if tr is not None:
            tr.update(norm2_out=h2, gate_proj=g_, up_proj=u_, silu_gate=sg, mlp_gated=gated,
                      down_res=d_res, resid_out=x.copy())
            tr["_f"].update(norm1_out=f_h, q_proj=f_q, k_proj=f_k, v_proj=f_v, q_rope=f_qr, k_rope=f_kr,
                            attn_ctx=f_c, norm2_out=f_h2, gate_proj=f_g, up_proj=f_u, silu_gate=f_s,
                            mlp_gated=f_m)                    # python/intref.py:284-285
        return x

    def final(self, x):                               # python/intref.py:296-301
        y = self.rmsnorm(x, (self.fg_q, self.fg_f), self.f_y, 16)
        acc = matmul_exact(y, self.wf("emb", self.emb_q), 1 << 15)
        return rs(acc * self.emb_m[None, :], self.emb_n + self.f_y - 16)

    def forward(self, ids, layers=NL, logits=True):
        """ids int64 [B, T] -> (embed [B,T,D], resid [layers,B,T,D], logits [B,T,V] or None)."""
        ids = np.asarray(ids, dtype=I64)
        if ids.ndim == 1:
            ids = ids[None, :]
        B, T = ids.shape
        x = self.embed(ids.reshape(-1))
        emb = x.copy()
        res = []
        for l in range(layers):
            x = self.block(l, x, T)
            res.append(x.copy())
        lg = self.final(x).reshape(B, T, V) if logits else None
        return emb.reshape(B, T, D), np.array(res).reshape(len(res), B, T, D), lg


def export_vectors(model, model_dir, ids, outdir, window=0):
    """Write ids.i64, exp_embed.i32, exp_resid_out.i32 [L,T,D], exp_logits.i32 [T,V] for one
    sequence (python/export_vectors.py:47-61) so c/intref.c can check them."""
    emb, res, lg = model.forward(ids[None, :])
    assert np.abs(lg).max() < 2 ** 31 and np.abs(res).max() < 2 ** 31   # export_vectors.py:58
    os.makedirs(outdir, exist_ok=True)
    np.asarray(ids, dtype=np.int64).tofile(os.path.join(outdir, "ids.i64"))
    emb[0].astype(np.int32).tofile(os.path.join(outdir, "exp_embed.i32"))
    res[:, 0].astype(np.int32).tofile(os.path.join(outdir, "exp_resid_out.i32"))
    lg[0].astype(np.int32).tofile(os.path.join(outdir, "exp_logits.i32"))
    return emb[0], res[:, 0], lg[0]
