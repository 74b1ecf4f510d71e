#!/usr/bin/env python3
"""Quantized-linear benchmark of the SAM 3 ViT on one MI355X through libsamhip.

Workload (one "step"): the K-quant sweep over the four SAM 3 ViT linear
shapes at M = 5184 tokens (a 72x72 patch grid): qkv 1024->3072, proj
1024->1024, fc1 1024->4736 in each of Q4_K, Q5_K and Q6_K, and fc2
4736->1024 in Q8_0 (4736 is not a multiple of 256, so every K-quant profile
stores fc2 as Q8_0: src/models/sam3/weights.hpp:159-160).  That is 12
mul_mat calls per step.  W ~ N(0, 0.02^2) (seed 0) packed on the device by
samhip_quantize_rows, X ~ N(0, 1) (seed 1), all resident in HBM before the
timed region.  Prints one JSON line.
"""

import argparse
import importlib.util
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
METRIC = "Q-matmul TOPS & % int8 MFMA peak; SAM3 Q4_K vision encode ms/image @1008px"
M_TOKENS = 5184
SHAPES = [("qkv", 1024, 3072), ("proj", 1024, 1024), ("fc1", 1024, 4736), ("fc2", 4736, 1024)]
PEAK_FP16_TFLOPS = 2500.0     # MI355X dense fp16 MFMA
PEAK_INT8_TOPS = 5000.0       # MI355X dense int8 MFMA
PEAK_HBM_GBPS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def load_samhip():
    path = os.path.join(ROOT, "sam.cpp_amd", "samhip.py")
    spec = importlib.util.spec_from_file_location("samhip", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def products(sh):
    """(label, weight type, K, N) of one step."""
    out = []
    for fmt in (sh.Q4_K, sh.Q5_K, sh.Q6_K):
        for name, k, n in SHAPES:
            qt = fmt if k % 256 == 0 else sh.Q8_0
            out.append((f"{name}:{sh.TYPE_NAMES[qt]}", qt, k, n))
    return out


def bytes_per_weight(sh, qt):
    return sh.BLOCK_BYTES[qt] / sh.BLOCK_ELEMS[qt]


def cpu_baseline(plan, seconds, rows):
    """The oracle's native-quantized CPU path (ggml-quantized-cpu-native-v1
    arithmetic, restated in C) on `rows` activation rows of every product."""
    sys.path.insert(0, ROOT)
    from oracle import oracle as O
    O.lib()
    threads = O.max_threads()
    rng = np.random.default_rng(1)
    xs = {k: rng.standard_normal((rows, k)).astype(np.float32) for _, _, k, _ in plan}
    ws = {}
    for label, qt, k, n in plan:
        w = (np.random.default_rng(0).standard_normal((n, k)) * 0.02).astype(np.float32)
        ws[label] = O.quantize(qt, w, O.ROUND_REF)
    ops, elapsed, passes = 0.0, 0.0, 0
    while elapsed < seconds and passes < 50:
        for label, qt, k, n in plan:
            t0 = time.perf_counter()
            O.mul_mat_native(qt, ws[label], xs[k], O.ROUND_X86, threads)
            elapsed += time.perf_counter() - t0
            ops += 2.0 * rows * n * k
        passes += 1
    return {"value": round(ops / elapsed / 1e12, 6), "unit": "TOPS", "cores": threads, "kind": "port",
            "sample": f"{rows} of {M_TOKENS} activation rows of each of the {len(plan)} products, {passes} passes, "
                      f"{elapsed:.1f} s; oracle/ggml_oracle.c native path (Q8_0/Q8_K activation packing + block "
                      f"integer dots), OpenMP"}


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--compute", choices=["native", "f16"], default="native")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--cpu-rows", type=int, default=96)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE {world}); the per-GPU shard is the single-GPU run.", file=sys.stderr)
        sys.exit(2)

    sh = load_samhip()
    compute = sh.COMPUTE_Q8_NATIVE if args.compute == "native" else sh.COMPUTE_F16
    ctx = sh.Context(0, compute, sh.ROUND_X86)
    plan = products(sh)

    log("preparing inputs")
    rng = np.random.default_rng(1)
    xbuf = {k: ctx.upload(rng.standard_normal((M_TOKENS, k)).astype(np.float32)) for k in sorted({p[2] for p in plan})}
    ops = []
    for label, qt, k, n in plan:
        wf = ctx.upload((np.random.default_rng(0).standard_normal((n, k)) * 0.02).astype(np.float32))
        wq = ctx.alloc(n * sh.row_bytes(qt, k))
        ctx.quantize_rows(qt, wf.ptr, 4 * k, wq.ptr, n, k, sh.ROUND_REF)
        ctx.synchronize()
        wf.free()
        yb = ctx.alloc(M_TOKENS * n * 4)
        w = sh.tensor(qt, k, n, wq.ptr)
        x = sh.tensor(sh.F32, k, M_TOKENS, xbuf[k].ptr)
        y = sh.tensor(sh.F32, n, M_TOKENS, yb.ptr)
        if not sh.lib().samhip_supports_mul_mat(w, x, y):
            raise RuntimeError(f"unsupported product {label}")
        ops.append((label, qt, k, n, w, x, y, wq, yb))

    def step():
        for _, _, _, _, w, x, y, _, _ in ops:
            ctx.mul_mat(w, x, y)

    for _ in range(args.warmup):
        step()
    ctx.synchronize()
    log(f"warmup done ({args.warmup} steps); timing {args.steps} steps")

    ctx.synchronize()
    ctx.trace_begin()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    records = ctx.trace_end(capacity=4 * len(ops) * args.steps + 16)   # waits for the stream
    elapsed = time.perf_counter() - t0
    log(f"timed {args.steps} steps in {elapsed * 1e3:.1f} ms")

    flops_step = sum(2.0 * M_TOKENS * n * k for _, _, k, n, *_ in ops)
    ms_step = elapsed * 1e3 / args.steps
    tops = flops_step * args.steps / elapsed / 1e12

    # per-kernel statistics from the HIP events on the launch stream
    by_kernel = {}
    for name, wt, m, n, k, ms in records:
        by_kernel.setdefault(name, []).append((m, n, k, ms))
    per_product = []
    for label, qt, k, n, *_ in ops:
        gname = [r for r in records if r[1] == qt and r[3] == n and r[4] == k and r[0].startswith("gemm")]
        sname = [r for r in records if r[1] == qt and r[3] == n and r[4] == k and r[0].startswith("stage")]
        g = float(np.mean([r[5] for r in gname])) if gname else float("nan")
        s = float(np.mean([r[5] for r in sname])) if sname else float("nan")
        per_product.append({"product": label, "M": M_TOKENS, "N": n, "K": k, "gemm_ms": round(g, 5),
                            "stage_ms": round(s, 5),
                            "gemm_tflops": round(2.0 * M_TOKENS * n * k / g / 1e9, 2),
                            "linear_tops": round(2.0 * M_TOKENS * n * k / (g + s) / 1e9, 2)})
    total = {name: sum(r[3] for r in rs) for name, rs in by_kernel.items()}
    dominant = max(total, key=total.get)
    launches = by_kernel[dominant]
    shapes = {(m, n, k) for m, n, k, _ in launches}
    m_, n_, k_ = max(shapes, key=lambda s: sum(r[3] for r in launches if r[:3] == s))
    same = [r[3] for r in launches if r[:3] == (m_, n_, k_)]
    avg_ms = float(np.mean(same))
    qt_dom = next(r[1] for r in records if r[0] == dominant)
    flops = 2.0 * m_ * n_ * k_
    achieved = flops / (avg_ms * 1e-3) / 1e12
    alg_bytes = n_ * k_ * bytes_per_weight(sh, qt_dom) + m_ * k_ * 2 + m_ * n_ * 4
    roofline = {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_FP16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_FP16_TFLOPS, 4), "traffic": None,
                "kernel": dominant, "shape": {"M": m_, "N": n_, "K": k_}, "launch_ms": round(avg_ms, 5),
                "launches": len(same), "flops_per_launch": flops,
                "algorithmic_bytes_per_launch": int(alg_bytes),
                "hbm_gbps_algorithmic": round(alg_bytes / (avg_ms * 1e-3) / 1e9, 1),
                "pct_int8_peak": round(100 * achieved / PEAK_INT8_TOPS, 2)}

    result = {
        "metric": METRIC, "value": round(tops, 3), "unit": "TOPS", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp16", "data": "synthetic",
        "config": {"workload": "SAM 3 ViT K-quant linear sweep (Q4_K/Q5_K/Q6_K qkv, proj, fc1; fc2 Q8_0) at "
                               "M=5184 tokens, 12 mul_mat per step",
                   "m_tokens": M_TOKENS, "compute": "q8-native" if compute == sh.COMPUTE_Q8_NATIVE else "f16",
                   "parallelism": "single-gpu", "activation": "F32 in HBM", "output": "F32"},
        "pct_int8_peak": round(100 * tops / PEAK_INT8_TOPS, 2),
        "roofline": roofline,
        "products": per_product,
        "device": ctx.query().device_name.decode(),
    }
    ctx.close()
    if not args.no_cpu_baseline:
        log("timing the CPU baseline")
        result["cpu_baseline"] = cpu_baseline([(p[0], p[1], p[2], p[3]) for p in ops], args.cpu_seconds, args.cpu_rows)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
