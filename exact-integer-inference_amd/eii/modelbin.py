"""The model.bin file ABI: sequential little-endian arrays, read and written here.

Layout (python/export_vectors.py:24-45, c/intref.c:8-13,70-91):

  header  emb_q int8[V*D], emb_m i64[V], emb_n i64[V], final_gain_q i64[D],
          final_gain_f i64, f_y i64, exp_table i64[DMAX+1],
          rope_cos i64[512*32], rope_sin i64[512*32]
  layer   fm i64[24] ((bits, f) for the 12 activation sites in SITES order),
  (x30)   ln1_q i64[D], ln1_f i64, ln2_q i64[D], ln2_f i64,
          q, k, v, o, gate, up, down: int8[N*K] (row = output channel), m i64[N], n i64[N],
          silu i64[65536]

The whole file is 154,045,048 bytes (the size pinned by vectors/t*/manifest.json).
"""
import os

import numpy as np

V, D, DFF, NH, NKV, HD, NL = 49152, 576, 1536, 9, 3, 64, 30
DMAX = 12 * 128
ROPE_POS = 512
F_RES, F_SCORE = 15, 7
EPS_S = 6184753
R_ISQRT = 40

SITES = ("norm1_out", "q_proj", "k_proj", "v_proj", "q_rope", "k_rope", "attn_ctx",
         "norm2_out", "gate_proj", "up_proj", "silu_gate", "mlp_gated")
MATS = ("q", "k", "v", "o", "gate", "up", "down")
MAT_NK = {"q": (576, 576), "k": (192, 576), "v": (192, 576), "o": (576, 576),
          "gate": (1536, 576), "up": (1536, 576), "down": (576, 1536)}

HEADER_BYTES = V * D + 2 * V * 8 + D * 8 + 8 + 8 + (DMAX + 1) * 8 + 2 * ROPE_POS * 32 * 8
LAYER_BYTES = (24 * 8 + 2 * (D * 8 + 8)
               + sum(n * k + 2 * n * 8 for n, k in MAT_NK.values()) + 65536 * 8)
FILE_BYTES = HEADER_BYTES + NL * LAYER_BYTES
assert FILE_BYTES == 154045048


def matrix_offset(layer, name):
    """Byte offset of matrix `name`'s int8 rows in layer `layer` (then m i64[N], n i64[N])."""
    off = HEADER_BYTES + layer * LAYER_BYTES + 24 * 8 + 2 * (D * 8 + 8)
    for m in MATS:
        if m == name:
            return off
        n, k = MAT_NK[m]
        off += n * k + 2 * n * 8
    raise KeyError(name)


class ModelBin:
    """Typed views over a model.bin image (a numpy memmap or an in-memory buffer).

    Attributes mirror the names the reference Model carries: emb_q/emb_m/emb_n, final_gain
    (q, f), f_y, exp_tab, rope_cos/rope_sin [512, 32], and layers[l] with fm [24], ln1/ln2
    (q, f), the seven matrices as (q int8 [N, K], m [N], n [N]) and silu [65536].
    """

    def __init__(self, buf):
        self.buf = buf
        off = 0

        def take(dtype, count):
            nonlocal off
            a = np.frombuffer(buf, dtype=dtype, count=count, offset=off)
            off += a.nbytes
            return a

        i64 = np.dtype("<i8")
        self.emb_q = take(np.int8, V * D).reshape(V, D)
        self.emb_m = take(i64, V)
        self.emb_n = take(i64, V)
        fg_q = take(i64, D)
        fg_f = int(take(i64, 1)[0])
        self.final_gain = (fg_q, fg_f)
        self.f_y = int(take(i64, 1)[0])
        self.exp_tab = take(i64, DMAX + 1)
        self.rope_cos = take(i64, ROPE_POS * 32).reshape(ROPE_POS, 32)
        self.rope_sin = take(i64, ROPE_POS * 32).reshape(ROPE_POS, 32)
        assert off == HEADER_BYTES
        self.layers = []
        for _ in range(NL):
            L = {"fm": take(i64, 24)}
            q1 = take(i64, D); f1 = int(take(i64, 1)[0])
            q2 = take(i64, D); f2 = int(take(i64, 1)[0])
            L["ln1"] = (q1, f1)
            L["ln2"] = (q2, f2)
            for name in MATS:
                n_, k_ = MAT_NK[name]
                q = take(np.int8, n_ * k_).reshape(n_, k_)
                m = take(i64, n_)
                n = take(i64, n_)
                L[name] = (q, m, n)
            L["silu"] = take(i64, 65536)
            self.layers.append(L)
        assert off == FILE_BYTES, (off, FILE_BYTES)

    def fmt(self, site, l):
        """(bits, f) of an activation site at layer l, as recorded in the layer's fm record."""
        i = SITES.index(site)
        fm = self.layers[l]["fm"]
        return int(fm[2 * i]), int(fm[2 * i + 1])


def read(path):
    size = os.path.getsize(path)
    if size != FILE_BYTES:
        raise ValueError(f"{path}: {size} bytes, a model.bin holds {FILE_BYTES}")
    return ModelBin(np.memmap(path, dtype=np.uint8, mode="r"))


def write(path, emb_q, emb_m, emb_n, final_gain, f_y, exp_tab, rope_cos, rope_sin, layers):
    """Write a model.bin in the byte order python/export_vectors.py:24-45 uses.

    layers[l] is a dict with fm (24 ints), ln1/ln2 (q, f), q..down as (q int8 [N,K], m, n) and silu.
    """
    def w(f, a, dt):
        f.write(np.ascontiguousarray(a, dtype=dt).tobytes())

    # A per-process temporary name: several processes may generate the same cached model at once
    # (parallel test workers); each renames its own complete file into place.
    tmp = "%s.%d.tmp" % (path, os.getpid())
    with open(tmp, "wb") as f:
        w(f, emb_q, np.int8); w(f, emb_m, "<i8"); w(f, emb_n, "<i8")
        w(f, final_gain[0], "<i8"); w(f, [final_gain[1]], "<i8"); w(f, [f_y], "<i8")
        w(f, exp_tab, "<i8")
        w(f, np.asarray(rope_cos)[:ROPE_POS], "<i8"); w(f, np.asarray(rope_sin)[:ROPE_POS], "<i8")
        for L in layers:
            w(f, L["fm"], "<i8")
            w(f, L["ln1"][0], "<i8"); w(f, [L["ln1"][1]], "<i8")
            w(f, L["ln2"][0], "<i8"); w(f, [L["ln2"][1]], "<i8")
            for name in MATS:
                q, m, n = L[name]
                assert q.shape == MAT_NK[name], (name, q.shape)
                w(f, q, np.int8); w(f, m, "<i8"); w(f, n, "<i8")
            w(f, L["silu"], "<i8")
    if os.path.getsize(tmp) != FILE_BYTES:
        raise ValueError("model.bin writer produced a file of the wrong size")
    os.replace(tmp, path)
