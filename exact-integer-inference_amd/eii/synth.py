"""Seeded synthetic SmolLM2-135M-shaped integer model and token ids.

The weights are random INT8 with per-row scales m * 2^-n (m in [2^13, 2^14]) in the
model.bin layout, with the reference's wide-mode format table (data/fm_wide.json) and
the exact exp/SiLU/RoPE tables.  Row shifts n are chosen per matrix from the output
format so that activations fill a few bits below their format's range, and every
bound the reference asserts holds (python/intref.py:49,61,189,259,279;
python/export_vectors.py:58): every requantization shift is >= 1 and |acc| * max m < 2^63.

Draw order from numpy.random.default_rng(seed) (PCG64), fixed for reproducibility:
  emb_q [V, D] int8 in [-127, 127]; emb_m [V] in [2^13, 2^14]; emb_n [V] in {20, 21, 22};
  final gain [D] in [2^13, 2^14) (f = 14); then per layer: ln1 gain [D], ln2 gain [D]
  (both f = 14), then for q, k, v, o, gate, up, down: q [N, K] int8 in [-127, 127],
  m [N] in [2^13, 2^14], n jitter [N] in {0, 1} added to the matrix's base shift.
"""
import math
import os

import numpy as np

from . import modelbin as mb
from .formats import load_fm
from .tables import exp_table, rope_tables, silu_table

# Configurations of the integer forward: (batch, tokens per sequence, window label).
# "window" only labels the data and seeds the ids (the reference's windows are indices
# into a token stream, python/export_vectors.py:17); attention is full causal.
CONFIGS = {
    "cfg1": dict(index=1, B=1, T=24, window=64),
    "cfg3": dict(index=3, B=1, T=128, window=64),
    "cfg4": dict(index=4, B=256, T=160, window=100),
    "cfg5": dict(index=5, B=32, T=4096, window=2048),
}
# sequences of cfg4 whose every state is checked against the oracle
CFG4_SAMPLED = (0, 37, 74, 111, 148, 185, 222, 255)
CFG5_SAMPLED = (0, 31)

GEMM_SHAPES = ((576, 576), (576, 192), (576, 1536), (1536, 576), (576, 49152))   # (K, N)
GEMM_M = 4096


def gemm_inputs(K, N, a_bits, M=GEMM_M):
    """The exact-matmul sweep's operands (python/intref.py:58-63 at the projection shapes): A [M, K]
    int16 or int32 with 99 % of the entries uniform in [-2^10, 2^10] and 1 % uniform over the
    whole type, the two extremes included; W int8 [N, K] uniform in [-127, 127].  Seeded by
    (K, N, a_bits)."""
    rng = np.random.default_rng([K, N, a_bits])
    dt = np.int16 if a_bits == 16 else np.int32
    info = np.iinfo(dt)
    A = rng.integers(-2 ** 10, 2 ** 10, size=(M, K), endpoint=True, dtype=np.int64)
    wide = rng.random((M, K)) < 0.01
    A[wide] = rng.integers(info.min, info.max, size=int(wide.sum()), endpoint=True, dtype=np.int64)
    A[0, 0], A[0, 1], A[M - 1, K - 1] = info.min, info.max, info.min
    W = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    return A.astype(dt), W


def token_ids(cfg):
    """int64 [B, T] token ids, uniform over the vocabulary, seeded by (config index, window)."""
    c = CONFIGS[cfg]
    rng = np.random.default_rng([c["index"], c["window"]])
    return rng.integers(0, mb.V, size=(c["B"], c["T"]), dtype=np.int64)


def _k_of(bits, f):
    return (bits - 1) - f


def _base_shift(K, sigma_in, sigma_out):
    # output std = sqrt(K) * sigma_in * 73.3 * E[m] * 2^-n * E[2^-jitter]
    g = math.sqrt(K) * sigma_in * (127 / math.sqrt(3)) * 12288 * 0.75 / sigma_out
    return int(round(math.log2(g)))


def make_layers(rng, fm, qk_boost=0):
    layers = []
    for l in range(mb.NL):
        f = fm[l]
        fmt = {s: (f[2 * i], f[2 * i + 1]) for i, s in enumerate(mb.SITES)}
        L = {"fm": list(f)}
        L["ln1"] = (rng.integers(1 << 13, 1 << 14, size=mb.D, dtype=np.int64), 14)
        L["ln2"] = (rng.integers(1 << 13, 1 << 14, size=mb.D, dtype=np.int64), 14)
        sig_norm = 0.76                                   # RMS of normalized value times gain
        k_v = _k_of(*fmt["v_proj"])
        sig_out = {
            "q": 2.0 ** (_k_of(*fmt["q_proj"]) - 4.5),     # scores of a few units: a spread softmax
            "k": 2.0 ** (_k_of(*fmt["k_proj"]) - 4.5),
            "v": 2.0 ** (k_v - 3.5),
            "o": 0.5,
            "gate": 2.0 ** (_k_of(*fmt["gate_proj"]) - 3.5),
            "up": 2.0 ** (_k_of(*fmt["up_proj"]) - 3.5),
            "down": 0.5,
        }
        sig_g = sig_out["gate"]
        sig_in = {"q": sig_norm, "k": sig_norm, "v": sig_norm, "gate": sig_norm, "up": sig_norm,
                  "o": 2.0 ** (k_v - 3.5) * 0.5,
                  "down": 0.5 * sig_g * sig_out["up"]}
        f_in = {"q": fmt["norm1_out"][1], "k": fmt["norm1_out"][1], "v": fmt["norm1_out"][1],
                "o": fmt["attn_ctx"][1], "gate": fmt["norm2_out"][1], "up": fmt["norm2_out"][1]}
        bits_s, f_s = fmt["silu_gate"]
        bits_m, f_m0 = fmt["mlp_gated"]
        f_u = fmt["up_proj"][1]
        f_in["down"] = min(f_m0, f_s + f_u) if bits_m == 32 else f_m0
        f_out = {"q": fmt["q_proj"][1], "k": fmt["k_proj"][1], "v": fmt["v_proj"][1],
                 "o": mb.F_RES, "gate": fmt["gate_proj"][1], "up": fmt["up_proj"][1], "down": mb.F_RES}
        for name in mb.MATS:
            N, K = mb.MAT_NK[name]
            q = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
            m = rng.integers(1 << 13, (1 << 14) + 1, size=N, dtype=np.int64)
            jit = rng.integers(0, 2, size=N, dtype=np.int64)
            base = _base_shift(K, sig_in[name], sig_out[name])
            if name in ("q", "k"):
                base -= qk_boost
            n = base + jit
            sh = n + f_in[name] - f_out[name]
            assert sh.min() >= 1, (l, name, int(sh.min()))
            L[name] = (q, m, n)
        bits_g, f_g = fmt["gate_proj"]
        L["silu"] = silu_table(f_g, f_s, bits_s)
        layers.append(L)
    return layers


def make_model(path, seed=0, qk_boost=0):
    """Write the seeded synthetic model to path (154,045,048 bytes)."""
    fm, f_y = load_fm()
    rng = np.random.default_rng(seed)
    emb_q = rng.integers(-127, 128, size=(mb.V, mb.D), dtype=np.int8)
    emb_m = rng.integers(1 << 13, (1 << 14) + 1, size=mb.V, dtype=np.int64)
    emb_n = rng.integers(20, 23, size=mb.V, dtype=np.int64)
    fg = (rng.integers(1 << 13, 1 << 14, size=mb.D, dtype=np.int64), 14)
    layers = make_layers(rng, fm, qk_boost)
    C, S = rope_tables(mb.ROPE_POS)
    mb.write(path, emb_q, emb_m, emb_n, fg, f_y, exp_table(), C, S, layers)
    return path


def default_model_path(kind="base"):
    """Cache location of the generated synthetic models (EII_MODEL_DIR, default ~/.cache/eii)."""
    d = os.environ.get("EII_MODEL_DIR", os.path.join(os.path.expanduser("~"), ".cache", "eii"))
    os.makedirs(d, exist_ok=True)
    return os.path.join(d, "model_seed0.bin" if kind == "base" else "model_seed0_qk4.bin")


def ensure_model(kind="base"):
    """Path of the synthetic model of this kind, generated on first use.

    kind "base": seed 0.  kind "stress": seed 0 with q/k row shifts lowered by 4, so q and k
    saturate their 16-bit formats and attention scores reach the ends of the softmax range.
    """
    p = default_model_path(kind)
    if not os.path.exists(p) or os.path.getsize(p) != mb.FILE_BYTES:
        make_model(p, seed=0, qk_boost=0 if kind == "base" else 4)
    return p


def rope_sidecar(T):
    """(cos, sin) int64 [T, 32] RoPE tables for positions beyond model.bin's 512 rows."""
    return rope_tables(T)


def make_float_checkpoint(path, seed=0):
    """A bfloat16 model.safetensors with the tensor names and shapes of SmolLM2-135M (the names
    python/common.py:50-68 reads) and random values at the real model's scales: matrices with
    standard deviation 1/sqrt(K), norm gains around 1.  Input of the real-weight path when the
    checkpoint itself is absent."""
    import torch
    from safetensors.torch import save_file
    g = torch.Generator().manual_seed(seed)

    def mat(n, k):
        return (torch.randn((n, k), generator=g) / math.sqrt(k)).to(torch.bfloat16)

    def gain(n):
        return (1.0 + 0.1 * torch.randn((n,), generator=g)).to(torch.bfloat16)

    t = {"model.embed_tokens.weight": mat(mb.V, mb.D), "model.norm.weight": gain(mb.D)}
    for l in range(mb.NL):
        p = f"model.layers.{l}."
        t[p + "input_layernorm.weight"] = gain(mb.D)
        t[p + "post_attention_layernorm.weight"] = gain(mb.D)
        for name, key in (("q", "self_attn.q_proj"), ("k", "self_attn.k_proj"), ("v", "self_attn.v_proj"),
                          ("o", "self_attn.o_proj"), ("gate", "mlp.gate_proj"), ("up", "mlp.up_proj"),
                          ("down", "mlp.down_proj")):
            t[p + key + ".weight"] = mat(*mb.MAT_NK[name])
    save_file(t, path)
    return path
