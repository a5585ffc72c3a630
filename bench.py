"""Throughput of the exact integer forward on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config cfg4]

A step is one full forward (embedding, 30 blocks, final norm, tied head with int32 logits)
over the configuration's whole batch of synthetic token ids, with the ids already in HBM.
Prints one JSON line.  The dominant kernel class is timed live with HIP events recorded on
its launch stream over the timed steps, and its roofline fraction is reported against the
int8 MFMA peak.  The CPU baseline runs the reference's own C program (c/intref.c, compiled
into oracle/_ref/intref by oracle/Makefile) on one sequence of the same workload, checking
the GPU's states at the same time; without that binary it times the numpy oracle instead.
"""
import argparse
import hashlib
import json
import os
import subprocess
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "exact-integer-inference_amd"))

import numpy as np

PEAK_INT8_OPS = 5.0e15          # MI355X dense int8 MFMA, ops/s
PEAK_HBM = 8.0e12               # bytes/s
V, D, DFF, NL = 49152, 576, 1536, 30
REF_BIN = os.path.join(ROOT, "oracle", "_ref", "intref")
GOLDEN = os.path.join(ROOT, "tests", "golden", "golden.json")
PROFILES = os.path.join(ROOT, "profiles")
COPY_BYTES = 1 << 30            # --copy-calibration: one plain device copy of 1 GiB


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def gemm_ops(engine, M):
    """Per-class (algorithmic ops, limb-weighted int8 MFMA ops) of one forward over M rows.

    Algorithmic ops are 2*M*N*K; the int8 MFMA executes one pass per limb of the activation
    (2 limbs for 16-bit inputs, 4 for 32-bit), so the MFMA work is 2*M*N*K*limbs."""
    ops = {k: [0.0, 0.0] for k in ("gemm_qkv", "gemm_o", "gemm_gate_up", "gemm_down", "gemm_head")}
    for l in range(NL):
        fm, _ = engine.formats(l)
        bits = {s: int(fm[2 * i]) for i, s in enumerate(
            ("norm1_out", "q_proj", "k_proj", "v_proj", "q_rope", "k_rope", "attn_ctx", "norm2_out",
             "gate_proj", "up_proj", "silu_gate", "mlp_gated"))}
        for k, N, K, site in (("gemm_qkv", 960, D, "norm1_out"), ("gemm_o", D, D, "attn_ctx"),
                              ("gemm_gate_up", 2 * DFF, D, "norm2_out"), ("gemm_down", D, DFF, "mlp_gated")):
            a = 2.0 * M * N * K
            ops[k][0] += a
            ops[k][1] += a * bits[site] // 8
    a = 2.0 * M * V * D
    ops["gemm_head"] = [a, 2 * a]
    return ops


def cpu_baseline_reference(model_path, ids, out):
    """Run the reference's C checker on sequence 0 with the GPU's states as the expected ones."""
    T = ids.shape[1]
    with tempfile.TemporaryDirectory() as d:
        ids[0].astype(np.int64).tofile(os.path.join(d, "ids.i64"))
        out["embed"][0].cpu().numpy().astype(np.int32).tofile(os.path.join(d, "exp_embed.i32"))
        out["resid"][:, 0].cpu().numpy().astype(np.int32).tofile(os.path.join(d, "exp_resid_out.i32"))
        out["logits"][0].cpu().numpy().astype(np.int32).tofile(os.path.join(d, "exp_logits.i32"))
        os.symlink(os.path.abspath(model_path), os.path.join(d, "model.bin"))
        t0 = time.perf_counter()
        r = subprocess.run([REF_BIN, d, d], capture_output=True, text=True, timeout=600)
        wall = time.perf_counter() - t0
    last = r.stdout.strip().splitlines()[-1] if r.stdout.strip() else ""
    cpu_s = wall
    if "(" in last and " s)" in last:
        cpu_s = float(last.split(",")[-1].split()[0])
    return {"value": T / cpu_s, "unit": "tokens/s", "cores": 1, "kind": "reference",
            "sample": f"1 sequence x {T} tokens of the benchmark batch (sequence 0), full 30-layer forward + "
                      f"head, reference c/intref.c -O2 on 1 host thread, its clock() CPU time",
            "seconds": cpu_s, "wall_seconds": wall, "verdict": last, "states_checked_by_reference": r.returncode == 0}


def measured_traffic(kernel, config):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 counter summary
    profiles/<kernel>_<config>_traffic.txt (FETCH_SIZE + WRITE_SIZE, scaled by the same counters
    on a plain copy of known size), or None when no summary exists for it."""
    path = os.path.join(PROFILES, f"{kernel}_{config}_traffic.txt")
    if not os.path.exists(path):
        return None
    vals = {}
    for line in open(path):
        if ":" in line and line.split(":")[0].strip() in ("fetch_bytes_per_launch", "write_bytes_per_launch"):
            vals[line.split(":")[0].strip()] = float(line.split(":")[1])
    if len(vals) != 2:
        return None
    return {"bytes": vals["fetch_bytes_per_launch"] + vals["write_bytes_per_launch"],
            "fetch": vals["fetch_bytes_per_launch"], "write": vals["write_bytes_per_launch"],
            "source": os.path.relpath(path, ROOT)}


def copy_calibration():
    """A plain device copy of COPY_BYTES, for scaling the HBM byte counters (run under rocprofv3)."""
    import torch
    src = torch.ones(COPY_BYTES, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": COPY_BYTES, "launches": 3}))


def cpu_baseline_port(model_path, ids):
    sys.path.insert(0, ROOT)
    from oracle.intref_np import OracleModel
    M = OracleModel(model_path)
    T = min(ids.shape[1], 64)
    t0 = time.perf_counter()
    M.forward(ids[:1, :T])
    s = time.perf_counter() - t0
    return {"value": T / s, "unit": "tokens/s", "cores": os.cpu_count(), "kind": "port",
            "sample": f"1 sequence x {T} tokens, numpy oracle (float64 BLAS exact products)", "seconds": s}


def gemm_sweep(args):
    """The exact-matmul sweep (eii_gemm_i8: int64 A W^T) at the projection shapes with 4096 rows of
    int32 and int16 activations; one JSON line with a record per shape and width.  Time = the
    whole operator (limb split of A, fragment order of W, the GEMM) per call, from events around
    --steps calls after --warmup.  Roofline: the int8 MFMA peak divided by the limb count, and
    8 TB/s over the algorithmic bytes (A, W, int64 output)."""
    import torch
    from eii import synth
    from eii import lib as L
    lib = L.load()
    recs = []
    for a_bits in (32, 16):
        for K, N in synth.GEMM_SHAPES:
            A, W = synth.gemm_inputs(K, N, a_bits)
            M = A.shape[0]
            At, Wt = torch.from_numpy(A).cuda(), torch.from_numpy(W).cuda()
            acc = torch.empty((M, N), dtype=torch.int64, device="cuda")
            wsum = torch.empty(N, dtype=torch.int32, device="cuda")
            L.check(lib.eii_weight_colsum(Wt.data_ptr(), N, K, wsum.data_ptr(), None))

            def call():
                L.check(lib.eii_gemm_i8_ws(At.data_ptr(), a_bits, Wt.data_ptr(), wsum.data_ptr(), M, N, K,
                                           acc.data_ptr(), None))
            for _ in range(args.warmup):
                call()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record()
            for _ in range(args.steps):
                call()
            e1.record()
            torch.cuda.synchronize()
            t = e0.elapsed_time(e1) * 1e-3 / args.steps
            limbs = a_bits // 8
            ops = 2.0 * M * N * K
            nbytes = (a_bits // 8) * M * K + N * K + 8 * M * N
            t_mfma, t_hbm = ops * limbs / 5.0e15, nbytes / 8.0e12
            recs.append({"K": K, "N": N, "a_bits": a_bits, "us": t * 1e6, "tops": ops / t / 1e12,
                         "gb_s": nbytes / t / 1e9, "mfma_frac": t_mfma / t, "hbm_frac": t_hbm / t,
                         "attainable_frac": max(t_mfma, t_hbm) / t, "bound": "mfma" if t_mfma > t_hbm else "hbm"})
            del At, Wt, acc
    print(json.dumps({"metric": "exact int64 matmul A W^T, 4096 rows (operator time incl. limb split)",
                      "unit": "per-shape records", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
                      "dtype": "int8", "data": "synthetic", "config": {"workload": "cfg2: (K, N) projection shapes",
                      "rows": synth.GEMM_M}, "results": recs}), flush=True)


def decode_bench(args):
    """KV-cached decoding over the configuration's batch: prompt = the first T - steps tokens,
    then steps appends of one token per sequence (the next token of the synthetic ids, so the
    logits equal those of the full forward), the last steps - warmup of them timed."""
    import torch
    from eii import synth
    from eii.engine import Engine
    ids_np = synth.token_ids(args.config)
    B, T = ids_np.shape
    n = args.steps
    if not 0 < args.warmup < n < T:
        raise SystemExit("--decode needs 0 < --warmup < --steps < tokens per sequence")
    eng = Engine(synth.ensure_model("stress" if args.config == "cfg5" else "base"), rope_rows=max(512, T))
    ids = torch.from_numpy(ids_np).cuda()
    kv = eng.kv_cache(B, T)
    try:
        kv.append(ids[:, :T - n], logits=False)
        for t in range(T - n, T - n + args.warmup):
            kv.append(ids[:, t:t + 1])
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for t in range(T - n + args.warmup, T):
            kv.append(ids[:, t:t + 1], check=False)
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        eng.check()
    finally:
        kv.close()
    steps = n - args.warmup
    print(json.dumps({"metric": "KV-cached decode tokens/s (one new token per sequence per step)",
                      "value": B * steps / elapsed, "unit": "tokens/s", "n_gpus": 1, "steps": steps,
                      "warmup": args.warmup, "ms_per_step": elapsed * 1e3 / steps, "higher_is_better": True,
                      "dtype": "int8", "data": "synthetic",
                      "config": {"workload": f"{args.config}: {B} sequences, {T - n}-token prompt, then single-token "
                                             f"appends with int32 logits [{B}, 1, {V}]", "batch": B}}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="cfg4")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 1 GiB device copy (the byte-counter calibration) and exit")
    ap.add_argument("--decode", action="store_true",
                    help="time KV-cached decoding instead: the configuration's sequences minus their last "
                         "--steps tokens as the prompt, then --steps single-token appends (one JSON line)")
    args = ap.parse_args()
    if args.copy_calibration:
        copy_calibration()
        return
    if args.decode:
        decode_bench(args)
        return
    if args.config == "cfg2":
        gemm_sweep(args)
        return
    if args.gpus != 1:
        print(f"bench.py: this engine runs on one GPU (sequences shard across GPUs with no exchange, "
              f"which this build does not launch); --gpus {args.gpus} is not supported", file=sys.stderr)
        sys.exit(2)

    import torch
    from eii import synth
    from eii.engine import Engine
    from eii import lib as L
    import ctypes as C

    cfg = synth.CONFIGS[args.config]
    kind = "stress" if args.config == "cfg5" else "base"
    model_path = synth.ensure_model(kind)
    ids_np = synth.token_ids(args.config)
    B, T = ids_np.shape
    M = B * T
    eng = Engine(model_path, rope_rows=max(512, T))
    ids = torch.from_numpy(ids_np).cuda()
    logits = torch.empty((M, V), dtype=torch.int32, device="cuda")
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    lib = eng.lib

    def step():
        L.check(lib.eii_forward(eng.h, C.c_void_p(ids.data_ptr()), B, T, None, None,
                                C.c_void_p(logits.data_ptr()), None, stream))

    for _ in range(args.warmup):
        step()
    eng.check()
    torch.cuda.synchronize()

    launches_per_step = 1 + NL * 9 + 2
    L.check(lib.eii_profile_begin(eng.h, launches_per_step * args.steps + 16))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms = (C.c_double * len(L.KERNEL_KINDS))()
    cnt = (C.c_int * len(L.KERNEL_KINDS))()
    L.check(lib.eii_profile_end(eng.h, stream, ms, cnt))
    eng.check()
    per_kind = {k: {"ms_total": ms[i], "launches": cnt[i]} for i, k in enumerate(L.KERNEL_KINDS)}

    tokens = M * args.steps
    value = tokens / elapsed
    ms_step = elapsed * 1e3 / args.steps

    ops = gemm_ops(eng, M)
    dom = max(ops, key=lambda k: per_kind[k]["ms_total"])
    t_dom = per_kind[dom]["ms_total"] * 1e-3 / args.steps           # seconds per step in this class
    n_dom = per_kind[dom]["launches"] / args.steps
    mfma_ops_launch = ops[dom][1] / n_dom
    avg_launch_s = t_dom / n_dom
    achieved = mfma_ops_launch / avg_launch_s
    fwd_mfma_ops = sum(v[1] for v in ops.values())

    # exactness of the timed workload: one more forward dumping the states of the sampled
    # sequences (and of sequence 0, which the CPU baseline checks), against the committed oracle
    # digests
    gold = {}
    if os.path.exists(GOLDEN):
        with open(GOLDEN) as f:
            gold = json.load(f).get(args.config, {}).get("sequences", {})
    dumped = sorted({0} | {int(b) for b in gold})
    out = eng.forward(ids_np, embed=True, resid=True, logits=True, dump=dumped)
    exact = None
    if gold:
        exact = True
        for b, g in gold.items():
            j = dumped.index(int(b))
            if (sha(out["resid"][:, j].cpu().numpy()) != g["resid_out"] or
                    sha(out["logits"][int(b)].cpu().numpy()) != g["logits"]):
                exact = False

    cpu = None
    if not args.no_cpu_baseline:
        if os.path.exists(REF_BIN) and T <= 512:
            cpu = cpu_baseline_reference(model_path, ids_np, out)
        else:
            cpu = cpu_baseline_port(model_path, ids_np)

    traffic = measured_traffic(dom, args.config)
    res = {
        "metric": "bit-exact tokens/s, 135M int fwd at B=256; int GEMM % of int8 MFMA peak",
        "value": value, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms_step, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8", "data": "synthetic",
        "config": {"workload": f"{args.config}: {B} independent sequences x {T} tokens, full 30-layer "
                               f"integer forward of the SmolLM2-135M shape + tied head (int32 logits)",
                   "batch": B, "tokens_per_sequence": T, "window_label": cfg["window"],
                   "weights": "seed-0 random int8 per-row-scaled, model.bin layout",
                   "parallelism": "single GPU"},
        "exact_sampled_sequences": exact,
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": achieved / 1e12, "peak": PEAK_INT8_OPS / 1e12,
                     "unit": "TFLOP/s", "frac": achieved / PEAK_INT8_OPS,
                     "traffic": traffic["bytes"] if traffic else None,
                     "traffic_detail": traffic,
                     "ops_per_launch_int8_mfma": mfma_ops_launch, "ops_per_launch_algorithmic": ops[dom][0] / n_dom,
                     "avg_launch_ms": avg_launch_s * 1e3},
        "forward_mfma_frac": fwd_mfma_ops / (elapsed / args.steps) / PEAK_INT8_OPS,
        "kernels_ms_per_step": {k: v["ms_total"] / args.steps for k, v in per_kind.items()},
        "cpu_baseline": cpu,
    }
    print(json.dumps(res))


if __name__ == "__main__":
    main()
