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
import collections
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
SWEEP_FORMATS = ("q4_K", "q5_K", "q6_K")   # weight formats of the sweep, in products() order
PEAK_FP16_TFLOPS = 2500.0     # MI355X dense fp16 MFMA
PEAK_INT8_TOPS = 5000.0       # MI355X dense int8 MFMA
PEAK_HBM_GBPS = 8000.0


# rocprofv3 commands whose CSV output summarize_profiles() reads
PROFILE_COMMANDS = {
    "trace": "rocprofv3 --kernel-trace --stats --output-format csv -d <out>/trace -o bench -- "
             "python3 bench.py --steps 50 --warmup 5 --no-cpu-baseline --no-encoder --no-configs",
    "text": "rocprofv3 --kernel-trace --stats --output-format csv -d <out>/text -o bench -- "
            "python3 bench.py --workload text --steps 10 --warmup 2",
    "encoder": "rocprofv3 --kernel-trace --stats --output-format csv -d <out>/encoder -o bench -- "
               "python3 bench.py --workload encoder --steps 5 --warmup 2 --no-cpu-baseline",
    "detector": "rocprofv3 --kernel-trace --stats --output-format csv -d <out>/detector -o bench -- "
                "python3 bench.py --workload detector --steps 10 --warmup 2",
    "fetch": "rocprofv3 --pmc FETCH_SIZE --output-format csv -d <out>/fetch -o bench -- "
             "python3 bench.py --steps 2 --warmup 1 --no-cpu-baseline --no-encoder --no-configs",
    "write": "rocprofv3 --pmc WRITE_SIZE --output-format csv -d <out>/write -o bench -- "
             "python3 bench.py --steps 2 --warmup 1 --no-cpu-baseline --no-encoder --no-configs",
    "pmc": "rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE SQ_BUSY_CYCLES "
           "SQ_WAIT_INST_LDS SQ_INSTS_LDS SQ_INSTS_MFMA GRBM_GUI_ACTIVE --output-format csv -d <out>/pmc -o bench -- "
           "python3 bench.py --steps 2 --warmup 1 --no-cpu-baseline --no-encoder --no-configs",
    "pmc2": "rocprofv3 --pmc SQ_ACTIVE_INST_VALU SQ_INSTS_VALU TCC_HIT_sum TCC_MISS_sum TCP_TCC_READ_REQ_LATENCY_sum "
            "TCP_TCC_READ_REQ_sum GRBM_GUI_ACTIVE --output-format csv -d <out>/pmc2 -o bench -- "
            "python3 bench.py --steps 2 --warmup 1 --no-cpu-baseline --no-encoder --no-configs",
    "copy_fetch": "rocprofv3 --pmc FETCH_SIZE --output-format csv -d <out>/copy_FETCH_SIZE -o copy -- "
                  "python3 bench.py --copy-calibration",
    "copy_write": "rocprofv3 --pmc WRITE_SIZE --output-format csv -d <out>/copy_WRITE_SIZE -o copy -- "
                  "python3 bench.py --copy-calibration",
}


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


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic_vit_sweep_m5184.json")
COPY_ELEMS = 1 << 26          # F32 elements of the calibration copy (256 MiB read + 256 MiB written)


def kernel_symbol(variant):
    """Template symbol of a GEMM variant name, as rocprofv3 reports it demangled:
    gemm_f16pipe_{BM}x{BN}x{BK}_s{S}[_w{WM}x{WN}]
        -> gemm_f16_pipe_kernel<BM, BN, BK, S, WM, WN, 0, 0> (2x2 waves by
           default; plain epilogue and A operand).
    Returns (symbol, threads per workgroup, BM, BN) or None."""
    import re
    m = re.fullmatch(r"gemm_f16pipe_(\d+)x(\d+)x(\d+)_s(\d+)(?:_w(\d+)x(\d+))?", variant)
    if m:
        bm, bn, bk, st = map(int, m.groups()[:4])
        wm, wn = (int(m.group(5)), int(m.group(6))) if m.group(5) else (2, 2)
        return f"gemm_f16_pipe_kernel<{bm}, {bn}, {bk}, {st}, {wm}, {wn}, 0, 0>", 64 * wm * wn, bm, bn
    return None


def hbm_traffic(variant, shape):
    """HBM bytes per launch of `variant` at `shape` = (M, N, K) from the
    committed FETCH_SIZE / WRITE_SIZE summary (each counter scaled by what it
    reads for a plain copy of known size), or None when not profiled."""
    sym = kernel_symbol(variant)
    if sym is None or not os.path.exists(TRAFFIC_FILE):
        return None
    symbol, threads, bm, bn = sym
    m, n, _ = shape
    grid = -(-m // bm) * -(-n // bn) * threads
    with open(TRAFFIC_FILE) as f:
        table = json.load(f)
    hits = [e["fetch_bytes"] + e["write_bytes"] for e in table["kernels"]
            if e["symbol"] == symbol and e["grid"] == grid and e.get("K") == shape[2]]
    return int(np.mean(hits)) if hits else None


def copy_calibration():
    """A plain streaming copy of known size (COPY_ELEMS F32 read, the same
    written) for scaling the FETCH_SIZE / WRITE_SIZE counters."""
    import torch
    x = torch.ones(COPY_ELEMS, device="cuda")
    torch.cuda.synchronize()
    y = x + 0.0
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": 4 * COPY_ELEMS, "copy_bytes_written": 4 * COPY_ELEMS,
                      "check": float(y[-1].item())}), flush=True)


def blas_calibration(iters=20):
    """hipBLASLt (torch.mm with an F32 output dtype) on fp16 operands at the
    four ViT product shapes (M = 5184), Y = A B^T with B row-major [N][K] as
    the staged weights are: the vendor library's time for the same operand
    formats and output type as this library's tall GEMM."""
    import torch
    out = {}
    for name, k, n in SHAPES:
        a = torch.randn(M_TOKENS, k, device="cuda", dtype=torch.float16)
        b = torch.randn(n, k, device="cuda", dtype=torch.float16)
        for _ in range(5):
            torch.mm(a, b.t(), out_dtype=torch.float32)
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(iters):
            torch.mm(a, b.t(), out_dtype=torch.float32)
        e.record()
        torch.cuda.synchronize()
        us = s.elapsed_time(e) / iters * 1e3
        out[name] = {"M": M_TOKENS, "N": n, "K": k, "us": round(us, 1),
                     "tflops": round(2.0 * M_TOKENS * n * k / (us * 1e-6) / 1e12, 1)}
    print(json.dumps({"hipblaslt_f16_f32out": out}), flush=True)


def summarize_profiles(d, commands):
    """Writes the committed text summaries from a rocprofv3 output folder
    `d` holding trace/, fetch/, write/, copy_FETCH_SIZE/ and copy_WRITE_SIZE/
    (CSV output of the commands listed in `commands`)."""
    import csv

    def rows(path):
        with open(path) as f:
            return list(csv.DictReader(f))

    def short(name):
        """`kernel<args>` from a demangled or Itanium-mangled kernel symbol
        (mangled names here carry only integer template arguments)."""
        import re
        m = re.match(r"_ZN6samhip12_GLOBAL__N_1(\d+)", name)
        if m:
            n = int(m.group(1))
            base = name[m.end():m.end() + n]
            rest = name[m.end() + n:]
            args = re.match(r"I((?:L[ib]-?\d+E)+)E", rest)
            if args:
                vals = [("true" if v == "1" else "false") if t == "b" else v
                        for t, v in re.findall(r"L([ib])(-?\d+)E", args.group(1))]
                base += "<" + ", ".join(vals) + ">"
            return base
        name = name.replace("void ", "", 1).replace("samhip::(anonymous namespace)::", "")
        return name.split("(")[0]

    def sweep_products(rs):
        """Dispatch id -> (product, K) for the sweep's dispatches: the sweep
        runs first and each mul_mat launches its preparation kernels and then
        one GEMM, in products() order, so the i-th GEMM dispatch is product
        i mod 12 (its grid must confirm it: proj and fc2 share a kernel and a
        grid) and a prep_kernel dispatch belongs to the GEMM that follows it.
        Products are named `shape:format` (fc2 is Q8_0 in every format)."""
        import re
        order = [(f"{name}:{'q8_0' if k % 256 else fmt}", name, k, n)
                 for fmt in SWEEP_FORMATS for name, k, n in SHAPES]
        by_id = {}
        for r in rs:
            by_id[int(r["Dispatch_Id"])] = (short(r["Kernel_Name"]), int(r.get("Grid_Size") or r["Grid_Size_X"]))
        out, pending, i = {}, [], 0
        for did in sorted(by_id):
            sym, grid = by_id[did]
            if sym.startswith("prep_kernel"):
                pending.append(did)
                continue
            if not sym.startswith("gemm_"):
                continue
            label, name, k, n = order[i % len(order)]
            t = re.match(r"gemm_f16_pipe_kernel<(\d+), (\d+), \d+, \d+, (\d+), (\d+)", sym)
            want = -(-M_TOKENS // int(t.group(1))) * -(-n // int(t.group(2))) * 64 * int(t.group(3)) * int(t.group(4)) \
                if t else None
            if want != grid:
                break
            for p_ in pending + [did]:
                out[p_] = (label, k)
            pending, i = [], i + 1
        if i % len(order):
            raise RuntimeError(f"{i} sweep GEMM dispatches matched: not whole steps of {len(order)}")
        return out

    copy_kib = {}
    for c in ("FETCH_SIZE", "WRITE_SIZE"):
        rs = [r for r in rows(os.path.join(d, f"copy_{c}", "copy_counter_collection.csv")) if "add" in r["Kernel_Name"]]
        copy_kib[c] = float(rs[0]["Counter_Value"])
    fetch_factor = 4 * COPY_ELEMS / 1024 / copy_kib["FETCH_SIZE"]
    write_factor = 4 * COPY_ELEMS / 1024 / copy_kib["WRITE_SIZE"]

    agg = {}
    for c, sub in (("FETCH_SIZE", "fetch"), ("WRITE_SIZE", "write")):
        rs = rows(os.path.join(d, sub, "bench_counter_collection.csv"))
        labels = sweep_products(rs)
        for r in rs:
            name, k = labels.get(int(r["Dispatch_Id"]), (None, None))
            key = (short(r["Kernel_Name"]), int(r["Grid_Size"]), name, k)
            agg.setdefault(key, {}).setdefault(c, []).append(float(r["Counter_Value"]))
    kernels = []
    for (sym, grid, name, k), v in sorted(agg.items(), key=lambda t: tuple(str(x) for x in t[0])):
        if "FETCH_SIZE" not in v or "WRITE_SIZE" not in v:
            continue
        fk = float(np.mean(v["FETCH_SIZE"]))
        wk = float(np.mean(v["WRITE_SIZE"]))
        kernels.append({"symbol": sym, "grid": grid, "product": name, "K": k, "dispatches": len(v["FETCH_SIZE"]),
                        "fetch_kib": round(fk, 1), "write_kib": round(wk, 1),
                        "fetch_bytes": int(fk * 1024 * fetch_factor), "write_bytes": int(wk * 1024 * write_factor)})
    table = {"fetch_factor": fetch_factor, "write_factor": write_factor, "copy_kib": copy_kib,
             "commands": commands, "kernels": kernels}
    os.makedirs(os.path.dirname(TRAFFIC_FILE), exist_ok=True)
    with open(TRAFFIC_FILE, "w") as f:
        json.dump(table, f, indent=1)

    def stats_table(sub, title, command, out_name, note=None):
        path = os.path.join(d, sub, "bench_kernel_stats.csv")
        if not os.path.exists(path):
            return
        # medians per kernel symbol from the same run's dispatch trace
        durations = {}
        trace = os.path.join(d, sub, "bench_kernel_trace.csv")
        if os.path.exists(trace):
            for r in rows(trace):
                durations.setdefault(short(r["Kernel_Name"]), []).append(
                    (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
        lines = [f"# {title}", "", "Command (from the repository root, `cd /tmp && export TMPDIR=/tmp` first):", "",
                 "```", command, "```", ""] + ([note, ""] if note else []) + [
                 "| kernel | calls | median us | avg us | min us | max us | share % |", "|---|---|---|---|---|---|---|"]
        for r in rows(path):
            ds = durations.get(short(r["Name"]))
            med = f"{float(np.median(ds)):.1f}" if ds else "-"
            lines.append(f"| `{short(r['Name'])}` | {r['Calls']} | {med} | {float(r['AverageNs']) / 1e3:.1f} | "
                         f"{float(r['MinNs']) / 1e3:.1f} | {float(r['MaxNs']) / 1e3:.1f} | {float(r['Percentage']):.1f} |")
        with open(os.path.join(ROOT, "profiles", out_name), "w") as f:
            f.write("\n".join(lines) + "\n")

    stats_table("trace", "Kernel time, SAM 3 ViT linear sweep at M=5184 (12 mul_mat per step)", commands["trace"],
                "kernel_stats_vit_sweep_m5184.md")
    trace_csv = os.path.join(d, "trace", "bench_kernel_trace.csv")
    if os.path.exists(trace_csv):
        rs = rows(trace_csv)
        labels = sweep_products(rs)
        per = {}
        for r in rs:
            did = int(r["Dispatch_Id"])
            if did not in labels:
                continue
            sym = short(r["Kernel_Name"])
            e = per.setdefault(labels[did][0], {"K": labels[did][1], "gemm": [], "prep": [], "symbol": None})
            us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
            if sym.startswith("gemm_"):
                e["gemm"].append(us)
                e["symbol"] = sym
            else:
                e["prep"].append(us)
        nmap = dict((nm, n) for nm, _, n in SHAPES)
        lines = ["", "Per product (same trace): every dispatch of the sweep is named by its product (each mul_mat "
                 "launches its preparation kernel and then one GEMM, in a fixed product order that each GEMM's grid "
                 "confirms). Medians and means over every step of the run, warmup included; the rates use the "
                 "medians.", "",
                 "| product | M | N | K | GEMM kernel | GEMM calls | GEMM median us | GEMM avg us | GEMM min us | "
                 "GEMM TFLOP/s | prep median us | linear TOPS |", "|---|---|---|---|---|---|---|---|---|---|---|---|"]
        seen = set()
        for label, _, k, n in [(f"{nm}:{'q8_0' if k_ % 256 else fmt}", nm, k_, n_)
                               for fmt in SWEEP_FORMATS for nm, k_, n_ in SHAPES]:
            e = per.get(label)
            if not e or not e["gemm"] or label in seen:
                continue
            seen.add(label)
            g, p_ = float(np.median(e["gemm"])), float(np.median(e["prep"])) if e["prep"] else 0.0
            fl = 2.0 * M_TOKENS * n * k
            lines.append(f"| {label} | {M_TOKENS} | {n} | {k} | `{e['symbol']}` | {len(e['gemm'])} | {g:.1f} | "
                         f"{float(np.mean(e['gemm'])):.1f} | {min(e['gemm']):.1f} | {fl / g / 1e6:.0f} | {p_:.1f} | "
                         f"{fl / (g + p_) / 1e6:.0f} |")
        with open(os.path.join(ROOT, "profiles", "kernel_stats_vit_sweep_m5184.md"), "a") as f:
            f.write("\n".join(lines) + "\n")
    stats_table("text", "Kernel time, SAM 3 text-encoder linear stream at M=32 (97 mul_mat per step, Q8_0)",
                commands["text"], "kernel_stats_text_stream_m32_q8_0.md")
    if os.path.isdir(os.path.join(d, "detector")):
        stats_table("detector", "Kernel time, SAM 3 fusion encoder + decoder linear stream (144 mul_mat per step, "
                    "Q8_0; image tokens M=5184, prompt M=33, queries M=201)", commands["detector"],
                    "kernel_stats_detector_stream_q8_0.md")
    stats_table("encoder", "Kernel time, SAM 3 vision encoder forward at 1008 px (Q4_K qkv/proj/fc1, Q8_0 fc2; "
                "8 forwards: 2 warmup, 5 timed, 1 traced)", commands["encoder"],
                "kernel_stats_vision_encoder_1008px_q4_k.md",
                note="`quantize_weights_kernel` and `quantize_act_kernel` pack the random-init weights once at set-up; "
                     "every other kernel runs 8 times per block (or per image for the prefix and the neck).  Template "
                     "arguments: `prep_kernel<mode, chunks, x86, weight type, pre>` (pre 1 = erf-GELU, 2 = layer "
                     "norm), `gemm_f16_pipe_kernel<BM, BN, BK, stages, waves M, waves N, epilogue, A operand>` "
                     "(epilogue bits 1 bias, 4 residual, 8 window unpartition, 16 packed attention operands, 32 "
                     "column scale, 64 transposed-convolution scatter, 128 erf-GELU; A operand 0 rows, 1 split rows "
                     "read as [hi | hi | lo], 2 gathered 3x3 convolution).")

    lines = ["# HBM traffic per dispatch, SAM 3 ViT linear sweep at M=5184", "",
             "Commands (from the repository root, `cd /tmp && export TMPDIR=/tmp` first):", "", "```",
             commands["fetch"], commands["write"], commands["copy_fetch"], commands["copy_write"], "```", "",
             f"Calibration: a plain copy of {4 * COPY_ELEMS} bytes (read, and the same written) reads "
             f"FETCH_SIZE {copy_kib['FETCH_SIZE']:.1f} KiB and WRITE_SIZE {copy_kib['WRITE_SIZE']:.1f} KiB, so "
             f"HBM bytes = FETCH_SIZE x 1024 x {fetch_factor:.3f} + WRITE_SIZE x 1024 x {write_factor:.3f}.", "",
             "Dispatches of the sweep are named by product (M 5184; each mul_mat launches its preparation kernel "
             "and then one GEMM, in a fixed product order that each GEMM's grid confirms); set-up kernels by "
             "grid.", "",
             "| kernel | grid (threads) | product | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | HBM MB read | "
             "HBM MB written |",
             "|---|---|---|---|---|---|---|---|"]
    nmap = dict((nm, n) for nm, _, n in SHAPES)
    for e in kernels:
        prod = f"{e['product']} N {nmap[e['product'].split(':')[0]]} K {e['K']}" if e["product"] else ""
        lines.append(f"| `{e['symbol']}` | {e['grid']} | {prod} | {e['dispatches']} | {e['fetch_kib']} | "
                     f"{e['write_kib']} | {e['fetch_bytes'] / 1e6:.2f} | {e['write_bytes'] / 1e6:.2f} |")
    with open(os.path.join(ROOT, "profiles", "hbm_traffic_vit_sweep_m5184.md"), "w") as f:
        f.write("\n".join(lines) + "\n")

    pmc_path = os.path.join(d, "pmc", "bench_counter_collection.csv")
    if os.path.exists(pmc_path):
        rs = rows(pmc_path)
        labels = sweep_products(rs)
        per = {}
        for r in rs:
            did = int(r["Dispatch_Id"])
            if did not in labels or not short(r["Kernel_Name"]).startswith("gemm_"):
                continue
            e = per.setdefault(did, {"symbol": short(r["Kernel_Name"]), "grid": int(r["Grid_Size"]),
                                     "product": labels[did],
                                     "us": (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3})
            e[r["Counter_Name"]] = e.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
        groups = {}
        for e in per.values():
            groups.setdefault((e["symbol"], e["grid"], e["product"]), []).append(e)
        lines = ["# MFMA and LDS counters, SAM 3 ViT linear sweep at M=5184 (GEMM kernels)", "",
                 "Command (from the repository root, `cd /tmp && export TMPDIR=/tmp` first):", "", "```",
                 commands["pmc"], "```", "",
                 "Medians per dispatch. MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 x 1024 SIMDs), "
                 "the profiler's own MFMA-utilization expression with GRBM_GUI_ACTIVE summed over the 8 XCD "
                 "instances; GUI_ACTIVE also counts cycles around the dispatch, so short kernels read low. LDS "
                 "conflict = SQ_LDS_BANK_CONFLICT / (SQ_LDS_IDX_ACTIVE - SQ_LDS_BANK_CONFLICT).", "",
                 "| kernel | grid (threads) | product | dispatches | dispatch us (under counters) | GUI_ACTIVE cycles "
                 "per XCD | MFMA busy % | LDS bank-conflict % | SQ_INSTS_MFMA | SQ_INSTS_LDS |",
                 "|---|---|---|---|---|---|---|---|---|---|"]
        for (sym, grid, (name, k)), es in sorted(groups.items(), key=lambda t: t[0][2][0]):
            def med(f):
                return float(np.median([f(e) for e in es]))
            gui = med(lambda e: e["GRBM_GUI_ACTIVE"] / 8)
            busy = med(lambda e: 100 * e["SQ_VALU_MFMA_BUSY_CYCLES"] / (e["GRBM_GUI_ACTIVE"] / 8 * 1024))
            conf = med(lambda e: 100 * e["SQ_LDS_BANK_CONFLICT"] /
                       max(1.0, e["SQ_LDS_IDX_ACTIVE"] - e["SQ_LDS_BANK_CONFLICT"]))
            lines.append(f"| `{sym}` | {grid} | {name} M {M_TOKENS} N {nmap[name.split(':')[0]]} K {k} | {len(es)} | "
                         f"{med(lambda e: e['us']):.1f} | {gui:.0f} | {busy:.1f} | {conf:.1f} | "
                         f"{med(lambda e: e['SQ_INSTS_MFMA']):.3g} | {med(lambda e: e['SQ_INSTS_LDS']):.3g} |")
        with open(os.path.join(ROOT, "profiles", "mfma_lds_counters_vit_sweep_m5184.md"), "w") as f:
            f.write("\n".join(lines) + "\n")

    pmc2_path = os.path.join(d, "pmc2", "bench_counter_collection.csv")
    if os.path.exists(pmc2_path):
        rs = rows(pmc2_path)
        labels = sweep_products(rs)
        per = {}
        for r in rs:
            did = int(r["Dispatch_Id"])
            sym = short(r["Kernel_Name"])
            if did not in labels or not (sym.startswith("gemm_") or sym.startswith("prep_")):
                continue
            e = per.setdefault(did, {"symbol": sym, "grid": int(r["Grid_Size"]), "product": labels[did],
                                     "us": (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3})
            e[r["Counter_Name"]] = e.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
        groups = {}
        for e in per.values():
            groups.setdefault((e["symbol"], e["grid"], e["product"]), []).append(e)
        lines = ["# L2 and VALU counters, SAM 3 ViT linear sweep at M=5184 (preparation and GEMM kernels)", "",
                 "Command (from the repository root, `cd /tmp && export TMPDIR=/tmp` first):", "", "```",
                 commands["pmc2"], "```", "",
                 "Medians per dispatch. L2 hit = TCC_HIT / (TCC_HIT + TCC_MISS) over all L2 channels. L2 read "
                 "latency = TCP_TCC_READ_REQ_LATENCY / TCP_TCC_READ_REQ: the mean cycles a vector L1 read request "
                 "waits for the L2 (hits and misses). VALU busy = SQ_ACTIVE_INST_VALU / (256 CUs x GRBM_GUI_ACTIVE "
                 "/ 8), the profiler's VALU-busy expression with GRBM_GUI_ACTIVE summed over the 8 XCD instances.",
                 "",
                 "| kernel | grid (threads) | product | dispatches | dispatch us (under counters) | L2 hit % | "
                 "L2 read latency (cycles) | VALU busy % | SQ_INSTS_VALU |",
                 "|---|---|---|---|---|---|---|---|---|"]
        for (sym, grid, (name, k)), es in sorted(groups.items(), key=lambda t: (t[0][2][0], t[0][0])):
            def med(f):
                return float(np.median([f(e) for e in es]))
            hit = med(lambda e: 100 * e["TCC_HIT_sum"] / max(1.0, e["TCC_HIT_sum"] + e["TCC_MISS_sum"]))
            lat = med(lambda e: e["TCP_TCC_READ_REQ_LATENCY_sum"] / max(1.0, e["TCP_TCC_READ_REQ_sum"]))
            valu = med(lambda e: 100 * e["SQ_ACTIVE_INST_VALU"] / (256 * e["GRBM_GUI_ACTIVE"] / 8))
            lines.append(f"| `{sym}` | {grid} | {name} M {M_TOKENS} N {nmap[name.split(':')[0]]} K {k} | {len(es)} | "
                         f"{med(lambda e: e['us']):.1f} | {hit:.1f} | {lat:.0f} | {valu:.1f} | "
                         f"{med(lambda e: e['SQ_INSTS_VALU']):.3g} |")
        with open(os.path.join(ROOT, "profiles", "l2_valu_counters_vit_sweep_m5184.md"), "w") as f:
            f.write("\n".join(lines) + "\n")


def cpu_info():
    """The host CPU model, the SIMD / matrix ISA extensions relevant to
    ggml's CPU kernels, and the thread settings (from /proc/cpuinfo and the
    environment)."""
    model, flags = None, set()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if model is None and line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                elif not flags and line.startswith("flags"):
                    flags = set(line.split(":", 1)[1].split())
    except OSError:
        pass
    isa = [x for x in ("sse4_2", "avx", "avx2", "fma", "f16c", "avx_vnni", "avx512f", "avx512bw", "avx512_vnni",
                       "avx512_bf16", "avx512_fp16", "amx_tile", "amx_int8", "amx_bf16") if x in flags]
    return {"model": model, "isa": isa, "nproc": os.cpu_count(), "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}


def cpu_baseline(plan, rows, samples=15, warmup=3):
    """Both CPU paths of the reference, restated in C by the oracle, on `rows`
    activation rows of every product (the protocol of the reference's probe,
    tools/benchmark/cpu_quantized_matmul_probe.cpp:43-67):
      native: ggml-quantized-cpu-native-v1 (activations packed to Q8_0 / Q8_K,
              block integer dots; src/runtime/ggml/runtime.hpp:105),
      decode: ggml-quantized-weights-f32-v1 (weights decoded to F32 per call,
              F32 dots; src/runtime/ggml/graph.hpp:111-139, runtime.hpp:106),
    each at all host cores and at 4 threads (the reference's default,
    include/sam/types.hpp:19): `warmup` untimed passes, then `samples`
    passes alternating the two paths AB/BA; median and P95 per pass."""
    sys.path.insert(0, ROOT)
    from oracle import oracle as O
    O.lib()
    all_threads = O.max_threads()
    rng = np.random.default_rng(1)
    xs = {k: rng.standard_normal((rows, k)).astype(np.float32) for _, _, k, _ in plan}
    ws = {}
    for label, qt, k, n in plan:
        w = (np.random.default_rng(0).standard_normal((n, k)) * 0.02).astype(np.float32)
        ws[label] = O.quantize(qt, w, O.ROUND_REF)
    ops = sum(2.0 * rows * n * k for _, _, k, n in plan)
    alg = sum(n * O.row_bytes(qt, k) + rows * k * 4 + rows * n * 4 for _, qt, k, n in plan)

    def one(path, threads):
        t0 = time.perf_counter()
        for label, qt, k, n in plan:
            if path == "native":
                O.mul_mat_native(qt, ws[label], xs[k], O.ROUND_X86, threads)
            else:
                O.mul_mat_decode(qt, ws[label], xs[k], threads)
        return time.perf_counter() - t0

    paths, spent = {}, 0.0
    for threads in sorted({all_threads, min(4, all_threads)}, reverse=True):
        for _ in range(warmup):
            spent += one("native", threads) + one("decode", threads)
        t = {"native": [], "decode": []}
        for i in range(samples):
            for p in (("native", "decode") if i % 2 == 0 else ("decode", "native")):
                t[p].append(one(p, threads))
                spent += t[p][-1]
        for p, v in t.items():
            med, p95 = float(np.median(v)), float(np.percentile(v, 95))
            paths[f"{p}_{threads}t"] = {"median_ms": round(med * 1e3, 3), "p95_ms": round(p95 * 1e3, 3),
                                        "tops": round(ops / med / 1e12, 6), "gbps": round(alg / med / 1e9, 3),
                                        "threads": threads, "samples": samples}
    # the value: the reference's default CPU policy (F32 decode), which is also
    # the faster of the two restated paths on these shapes
    head = paths[f"decode_{all_threads}t"]
    return {"value": head["tops"], "unit": "TOPS", "cores": all_threads, "kind": "port",
            "sample": f"{rows} of {M_TOKENS} activation rows of each of the {len(plan)} products per pass; "
                      f"{warmup} warmup + {samples} timed passes per path, AB/BA alternated, at {all_threads} and "
                      f"4 threads ({spent:.1f} s); value = F32-decode path (the reference's default CPU policy), "
                      f"all threads, median; oracle/ggml_oracle.c restating ggml's CPU arithmetic (ggml itself "
                      f"is not available: its SIMD kernels are not reproduced), OpenMP",
            "paths": paths, "host": cpu_info()}


def stream_cpu_baseline(shape_counts, qt, seconds=10.0):
    """The oracle's native-quantized CPU path on every distinct (M, N, K) of a
    linear stream, each timed once per pass, the stream's time being the sum
    over shapes of time x occurrences; reported as algorithmic GB/s like the
    GPU line."""
    sys.path.insert(0, ROOT)
    from oracle import oracle as O
    O.lib()
    threads = O.max_threads()
    rb = {k: O.row_bytes(qt, k) for _, _, k in shape_counts}
    data = {}
    for m, n, k in shape_counts:
        w = (np.random.default_rng(0).standard_normal((n, k)) * 0.02).astype(np.float32)
        data[(m, n, k)] = (O.quantize(qt, w, O.ROUND_REF),
                           np.random.default_rng(1).standard_normal((m, k)).astype(np.float32))
    times = {key: 0.0 for key in shape_counts}
    passes, spent = 0, 0.0
    while spent < seconds and passes < 20:
        for key, (w, x) in data.items():
            t0 = time.perf_counter()
            O.mul_mat_native(qt, w, x, O.ROUND_X86, threads)
            dt = time.perf_counter() - t0
            times[key] += dt
            spent += dt
        passes += 1
    stream_s = sum(times[key] / passes * cnt for key, cnt in shape_counts.items())
    alg = sum((n * rb[k] + m * k * 4 + m * n * 4) * cnt for (m, n, k), cnt in shape_counts.items())
    return {"value": round(alg / stream_s / 1e9, 2), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"each of the {len(shape_counts)} distinct (M, N, K) of the stream timed {passes} times "
                      f"({spent:.1f} s), weighted by its {sum(shape_counts.values())} occurrences; "
                      f"oracle/ggml_oracle.c native path, OpenMP"}


TEXT_LAYERS = 24
TEXT_M = 32
TEXT_SHAPES = [("in_proj", 1024, 3072), ("out_proj", 1024, 1024), ("fc1", 1024, 4096), ("fc2", 4096, 1024)]


def text_stream(args, sh, ctx, fmt):
    """The text encoder's linear stream at M = 32 tokens: 24 layers of
    in_proj 1024->3072, out_proj 1024->1024, fc1 1024->4096, fc2 4096->1024
    and the resizer 1024->256 (src/models/sam3/text_encoder.hpp:83-174), 97
    mul_mat per step, every layer with its own weight buffers so that the
    stream's weights (321 MB in Q8_0) pass through HBM as they do in the
    model.  The timed steps replay the stream captured as one HIP graph (the
    eager per-call time is reported beside it).  One JSON line: algorithmic
    bytes (packed W + F32 X + F32 Y) per second over the whole stream, and
    the skinny kernel's roofline."""
    qt = {"q8_0": sh.Q8_0, "q4_k": sh.Q4_K, "q5_k": sh.Q5_K, "q6_k": sh.Q6_K}[fmt]
    log("preparing text stream weights")
    rng = np.random.default_rng(1)
    xbuf = {k: ctx.upload(rng.standard_normal((TEXT_M, k)).astype(np.float32)) for k in (1024, 4096)}
    shapes = [(f"L{l}.{name}", k, n) for l in range(TEXT_LAYERS) for name, k, n in TEXT_SHAPES]
    shapes.append(("resizer", 1024, 256))
    packed = {}
    for name, k, n in set((nm.split(".")[-1], k, n) for nm, k, n in shapes):
        wf = ctx.upload((np.random.default_rng(0).standard_normal((n, k)) * 0.02).astype(np.float32))
        packed[(k, n)] = wf
    ops, alg_bytes = [], 0
    for label, k, n in shapes:
        wq = ctx.alloc(n * sh.row_bytes(qt, k))
        ctx.quantize_rows(qt, packed[(k, n)].ptr, 4 * k, wq.ptr, n, k, sh.ROUND_REF)
        yb = ctx.alloc(TEXT_M * n * 4)
        ops.append((label, k, n, sh.tensor(qt, k, n, wq.ptr), sh.tensor(sh.F32, k, TEXT_M, xbuf[k].ptr),
                    sh.tensor(sh.F32, n, TEXT_M, yb.ptr), wq, yb))
        alg_bytes += n * sh.row_bytes(qt, k) + TEXT_M * k * 4 + TEXT_M * n * 4
    ctx.synchronize()
    for wf in packed.values():
        wf.free()

    def step():
        for _, _, _, w, x, y, _, _ in ops:
            ctx.mul_mat(w, x, y)

    for _ in range(args.warmup):
        step()
    ctx.trace_begin()
    step()
    prof = ctx.trace_end(capacity=4 * len(ops) + 16)
    ctx.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    ctx.synchronize()
    eager = time.perf_counter() - t0
    # the same stream captured once and replayed: one host call per step
    ctx.capture_begin()
    step()
    graph = ctx.capture_end()
    graph.launch()
    ctx.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        graph.launch()
    ctx.synchronize()
    elapsed = time.perf_counter() - t0
    graph.destroy()
    kern = [r for r in prof if r[0].startswith("skinny")]
    stage = [r for r in prof if r[0].startswith("stage")]
    fc1 = [r[5] for r in kern if r[3] == 4096 and r[4] == 1024]
    fc1_ms = float(np.mean(fc1))
    fc1_bytes = 4096 * sh.row_bytes(qt, 1024) + TEXT_M * 1024 * 4 + TEXT_M * 4096 * 4
    ach = fc1_bytes / (fc1_ms * 1e-3) / 1e9
    return {
        "metric": "text linear stream algorithmic GB/s (M=32, 24 layers)", "value": round(alg_bytes * args.steps / elapsed / 1e9, 1),
        "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(elapsed * 1e3 / args.steps, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp16", "data": "synthetic",
        "config": {"workload": f"SAM 3 text encoder linear stream, {fmt.upper()} weights, M=32 tokens, 97 mul_mat per step",
                   "weights_mb": round(sum(o[6].nbytes for o in ops) / 1e6, 1), "parallelism": "single-gpu"},
        "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": round(ach / PEAK_HBM_GBPS, 4), "traffic": None, "kernel": kern[0][0] if kern else None,
                     "shape": {"M": TEXT_M, "N": 4096, "K": 1024}, "launch_ms": round(fc1_ms, 5),
                     "algorithmic_bytes_per_launch": int(fc1_bytes)},
        "eager_ms_per_step": round(eager * 1e3 / args.steps, 4),
        "cpu_baseline": None if args.no_cpu_baseline else stream_cpu_baseline(
            collections.Counter((TEXT_M, n, k) for _, k, n in shapes), qt, args.cpu_seconds),
        "replay": "one HIP graph launch per step (samhip_capture_begin/end)",
        "kernel_ms_per_step": round(sum(r[5] for r in kern), 4),
        "stage_ms_per_step": round(sum(r[5] for r in stage), 4),
        "device": ctx.query().device_name.decode(),
    }


DET_D, DET_FFN, DET_LAYERS = 256, 2048, 6
DET_M = {"img": 5184, "prompt": 33, "query": 201}


def detector_plan():
    """The linears of the fusion encoder (src/models/sam3/fusion_encoder.hpp:46-145) and of the DETR
    decoder (src/models/sam3/detector.hpp:343-479), 6 layers each, D = 256, FFN 2048.  Entries:
    (label, weight key, weight rows, row offset, N, K, activation key).  q/k/v are row-offset views of
    the fused [3D, D] in-projections, as the reference takes them with ggml_view_2d."""
    D, F = DET_D, DET_FFN
    plan = []
    for l in range(DET_LAYERS):
        f = f"fenc{l}"
        for i, (part, src) in enumerate((("q", "img"), ("k", "img"), ("v", "img"))):
            plan.append((f"{f}.sa_{part}", f"{f}.sa_in", 3 * D, i * D, D, D, (src, D)))
        plan.append((f"{f}.sa_out", f"{f}.sa_out", D, 0, D, D, ("img", D)))
        for i, (part, src) in enumerate((("q", "img"), ("k", "prompt"), ("v", "prompt"))):
            plan.append((f"{f}.ca_{part}", f"{f}.ca_in", 3 * D, i * D, D, D, (src, D)))
        plan.append((f"{f}.ca_out", f"{f}.ca_out", D, 0, D, D, ("img", D)))
        plan.append((f"{f}.fc1", f"{f}.fc1", F, 0, F, D, ("img", D)))
        plan.append((f"{f}.fc2", f"{f}.fc2", D, 0, D, F, ("img", F)))
    for l in range(DET_LAYERS):
        d = f"ddec{l}"
        for i, part in enumerate("qkv"):
            plan.append((f"{d}.sa_{part}", f"{d}.sa_in", 3 * D, i * D, D, D, ("query", D)))
        plan.append((f"{d}.sa_out", f"{d}.sa_out", D, 0, D, D, ("query", D)))
        for ca, kv in (("ca_text", "prompt"), ("ca_img", "img")):
            for i, (part, src) in enumerate((("q", "query"), ("k", kv), ("v", kv))):
                plan.append((f"{d}.{ca}_{part}", f"{d}.{ca}_in", 3 * D, i * D, D, D, (src, D)))
            plan.append((f"{d}.{ca}_out", f"{d}.{ca}_out", D, 0, D, D, ("query", D)))
        plan.append((f"{d}.fc1", f"{d}.fc1", F, 0, F, D, ("query", D)))
        plan.append((f"{d}.fc2", f"{d}.fc2", D, 0, D, F, ("query", F)))
    return plan


def detector_stream(args, sh, ctx, fmt):
    """Config 3's fusion and decoder half: the 6 fusion-encoder and 6 decoder layers' linears (image
    tokens M = 5184, prompt tokens M = 33, queries M = 201; D = 256, FFN 2048), every layer with its
    own weights and the q/k/v products on row-offset views of the fused in-projections, 144 mul_mat
    per step replayed as one HIP graph.  One JSON line: algorithmic bytes (packed W + F32 X + F32 Y)
    per second over the stream, its TOPS, per-shape times, and the dominant kernel's roofline."""
    qt = {"q8_0": sh.Q8_0, "q4_k": sh.Q4_K, "q5_k": sh.Q5_K, "q6_k": sh.Q6_K}[fmt]
    log("preparing fusion/decoder stream weights")
    plan = detector_plan()
    rng = np.random.default_rng(3)
    xbuf = {(src, k): ctx.upload(rng.standard_normal((DET_M[src], k)).astype(np.float32))
            for src, k in sorted({p[6] for p in plan})}
    wbuf = {}
    for _, key, rows, _, _, k, _ in plan:
        if key in wbuf:
            continue
        wf = ctx.upload((np.random.default_rng(len(wbuf)).standard_normal((rows, k)) * 0.02).astype(np.float32))
        wq = ctx.alloc(rows * sh.row_bytes(qt, k))
        ctx.quantize_rows(qt, wf.ptr, 4 * k, wq.ptr, rows, k, sh.ROUND_REF)
        ctx.synchronize()
        wf.free()
        wbuf[key] = wq
    ops, alg_bytes, flops = [], 0, 0
    for label, key, rows, off, n, k, (src, _) in plan:
        m, rb = DET_M[src], sh.row_bytes(qt, k)
        yb = ctx.alloc(m * n * 4)
        w = sh.tensor(qt, k, n, wbuf[key].ptr + off * rb, nb1=rb)
        x = sh.tensor(sh.F32, k, m, xbuf[(src, k)].ptr)
        y = sh.tensor(sh.F32, n, m, yb.ptr)
        if not sh.lib().samhip_supports_mul_mat(w, x, y):
            raise RuntimeError(f"unsupported product {label}")
        ops.append((label, m, n, k, w, x, y, yb))
        alg_bytes += n * rb + m * k * 4 + m * n * 4
        flops += 2 * m * n * k

    def step():
        for _, _, _, _, w, x, y, _ in ops:
            ctx.mul_mat(w, x, y)

    for _ in range(args.warmup):
        step()
    ctx.trace_begin()
    step()
    prof = ctx.trace_end(capacity=4 * len(ops) + 16)
    ctx.synchronize()
    ctx.capture_begin()
    step()
    graph = ctx.capture_end()
    graph.launch()
    ctx.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        graph.launch()
    ctx.synchronize()
    elapsed = time.perf_counter() - t0
    graph.destroy()
    # per (M, N, K) shape: launches and event time per step
    shapes = {}
    for name, _, m, n, k, ms in prof:
        e = shapes.setdefault((m, n, k), {"M": m, "N": n, "K": k, "ms": 0.0, "kernels": {}})
        e["ms"] += ms
        e["kernels"][name] = e["kernels"].get(name, 0) + 1
    per_kernel = {}
    for name, _, m, n, k, ms in prof:
        per_kernel[name] = per_kernel.get(name, 0.0) + ms
    dom = max(per_kernel, key=per_kernel.get)
    dom_recs = [(m, n, k, ms) for name, _, m, n, k, ms in prof if name == dom]
    rb_of = {k: sh.row_bytes(qt, k) for k in (DET_D, DET_FFN)}
    dom_bytes = sum(n * rb_of[k] + m * k * 4 + m * n * 4 for m, n, k, _ in dom_recs)
    dom_ms = sum(r[3] for r in dom_recs)
    ach = dom_bytes / (dom_ms * 1e-3) / 1e9
    for b in list(wbuf.values()) + list(xbuf.values()) + [o[7] for o in ops]:
        b.free()
    return {
        "metric": "fusion/decoder linear stream algorithmic GB/s (D=256, 6+6 layers)",
        "value": round(alg_bytes * args.steps / elapsed / 1e9, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(elapsed * 1e3 / args.steps, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16", "data": "synthetic",
        "config": {"workload": f"SAM 3 fusion encoder + decoder linear stream, {fmt.upper()} weights, image tokens "
                               f"M=5184, prompt M=33, queries M=201, {len(ops)} mul_mat per step",
                   "parallelism": "single-gpu"},
        "tops": round(flops * args.steps / elapsed / 1e12, 2),
        "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": round(ach / PEAK_HBM_GBPS, 4), "traffic": None, "kernel": dom,
                     "launches": len(dom_recs), "launch_ms": round(dom_ms / len(dom_recs), 5)},
        "shapes": sorted(({**e, "ms": round(e["ms"], 4)} for e in shapes.values()), key=lambda e: -e["ms"]),
        "cpu_baseline": None if args.no_cpu_baseline else stream_cpu_baseline(
            collections.Counter((DET_M[p[6][0]], p[4], p[5]) for p in plan), qt, args.cpu_seconds),
        "replay": "one HIP graph launch per step (samhip_capture_begin/end)",
        "device": ctx.query().device_name.decode(),
    }


ENC = {"E": 1024, "HEADS": 16, "MLP": 4736, "GRID": 72, "WINDOW": 24, "IMG": 1008, "PATCH": 14, "POS_GRID": 24,
       "DEPTH": 32, "GLOBAL": (7, 15, 23, 31), "NECK_MID": 512, "NECK_DIM": 256}


def neck_flops(grid, E, mid, D):
    """Algorithmic flops of neck levels 0-2 (2 per multiply-add)."""
    T = grid * grid
    mac = (T * E * 4 * mid + 4 * T * mid * 4 * D + 16 * T * D * D + 16 * T * 9 * D * D   # level 0
           + T * E * 4 * mid + 4 * T * mid * D + 4 * T * 9 * D * D                      # level 1
           + T * E * D + T * 9 * D * D)                                                 # level 2
    return 2.0 * mac


def axial_rope_table(width, height, hd, theta=10000.0):
    """Axial 2-D RoPE table (cos, sin) [width*height][hd/2][2]: hd/4
    frequencies per axis, token t = y*width + x.  A converted checkpoint
    carries its own table (vit.blocks.N.attn.freqs_cis); any unit-modulus
    table costs the same."""
    freqs = 1.0 / theta ** (np.arange(0, hd, 4)[: hd // 4].astype(np.float64) / hd)
    t = np.arange(width * height)
    ang = np.concatenate([np.outer(t % width, freqs), np.outer(t // width, freqs)], axis=1)
    return np.stack([np.cos(ang), np.sin(ang)], axis=-1).astype(np.float32)


class Encoder:
    """A random-init SAM 3 vision encoder on the device (1008 px, 72x72
    tokens, width 1024, 32 pre-LN blocks, 16 heads, MLP 4736, window 24 with
    global attention in blocks 7/15/23/31) and its SimpleFPN neck (mid 512,
    dim 256; levels 0-2 as the image path outputs them, F32 columns):
    qkv/proj/fc1 in the K-quant `qt`, fc2 in Q8_0 (4736-wide rows),
    norms/biases/embeddings/neck F32.  Linear weights N(0, 0.02^2) packed on
    the device by samhip_quantize_rows."""

    def __init__(self, sh, ctx, qt, seed=0):
        import ctypes
        self.sh, self.ctx, self.ctypes = sh, ctx, ctypes
        e = ENC
        E, H, MLP, G, WS = e["E"], e["HEADS"], e["MLP"], e["GRID"], e["WINDOW"]
        rng = np.random.default_rng(seed)
        self.keep, self.blocks = [], []
        tables = {False: ctx.upload(axial_rope_table(WS, WS, E // H)), True: ctx.upload(axial_rope_table(G, G, E // H))}
        self.keep += list(tables.values())

        def f32(a):
            b = ctx.upload(np.ascontiguousarray(a, np.float32))
            self.keep.append(b)
            return b.ptr

        def packed(t, n, k):
            wf = ctx.upload((rng.standard_normal((n, k), dtype=np.float32) * 0.02))
            wq = ctx.alloc(n * sh.row_bytes(t, k))
            ctx.quantize_rows(t, wf.ptr, 4 * k, wq.ptr, n, k, sh.ROUND_REF)
            ctx.synchronize()
            wf.free()
            self.keep.append(wq)
            return sh.tensor(t, k, n, wq.ptr)

        for i in range(e["DEPTH"]):
            glob = i in e["GLOBAL"]
            d = sh.VitBlockDesc()
            d.version = sh.ABI_VERSION
            d.embed, d.heads, d.mlp, d.grid_w, d.grid_h, d.window = E, H, MLP, G, G, 0 if glob else WS
            d.norm1_w, d.norm2_w = f32(1 + 0.1 * rng.standard_normal(E)), f32(1 + 0.1 * rng.standard_normal(E))
            d.norm1_b, d.norm2_b = f32(0.05 * rng.standard_normal(E)), f32(0.05 * rng.standard_normal(E))
            d.qkv_b, d.proj_b = f32(0.02 * rng.standard_normal(3 * E)), f32(0.02 * rng.standard_normal(E))
            d.fc1_b, d.fc2_b = f32(0.02 * rng.standard_normal(MLP)), f32(0.02 * rng.standard_normal(E))
            d.freqs_cis = tables[glob].ptr
            d.qkv_w, d.proj_w = packed(qt, 3 * E, E), packed(qt, E, E)
            d.fc1_w, d.fc2_w = packed(qt, MLP, E), packed(sh.Q8_0, E, MLP)
            self.blocks.append(d)
        self.prefix = sh.VitPrefix(ctx, rng.standard_normal((E, 3, e["PATCH"], e["PATCH"]), dtype=np.float32) * 0.02,
                                   rng.standard_normal((e["POS_GRID"], e["POS_GRID"], E), dtype=np.float32) * 0.1,
                                   1 + 0.1 * rng.standard_normal(E), 0.05 * rng.standard_normal(E), e["IMG"],
                                   e["PATCH"], E, e["POS_GRID"])
        self.image = ctx.upload(np.random.default_rng(seed + 1).standard_normal((3, e["IMG"], e["IMG"]), dtype=np.float32))
        self.x = ctx.alloc(G * G * E * 4)
        mid, D = e["NECK_MID"], e["NECK_DIM"]
        nr = np.random.default_rng(seed + 2)

        def nw(*shape):
            return (nr.standard_normal(shape, dtype=np.float32) * 0.02).ravel()
        # oracle-keyed (or_neck_weights) host copies, ggml layouts
        self.neck_host = {"s0_dc1_w": nw(E, mid, 2, 2), "s0_dc1_b": nw(mid), "s0_dc2_w": nw(mid, D, 2, 2),
                          "s0_dc2_b": nw(D), "s0_c1_w": nw(D, D), "s0_c1_b": nw(D), "s0_c3_w": nw(D, D, 3, 3),
                          "s0_c3_b": nw(D), "s1_dc_w": nw(E, mid, 2, 2), "s1_dc_b": nw(mid), "s1_c1_w": nw(D, mid),
                          "s1_c1_b": nw(D), "s1_c3_w": nw(D, D, 3, 3), "s1_c3_b": nw(D), "s2_c1_w": nw(D, E),
                          "s2_c1_b": nw(D), "s2_c3_w": nw(D, D, 3, 3), "s2_c3_b": nw(D)}
        keys = {"dc1": "deconv1", "dc": "deconv1", "dc2": "deconv2", "c1": "conv1x1", "c3": "conv3x3"}
        scales = [{}, {}, {}, {}]
        for name, v in self.neck_host.items():
            lv, part, kind = name.split("_")
            scales[int(lv[1])][f"{keys[part]}_{kind}"] = v
        self.neck = sh.VitNeck(ctx, scales, G, E, mid, D, sh.F32)
        self.levels = [ctx.alloc(self.neck.level_rows(i) * D * 4) for i in range(3)] + [None]
        self.flops = self._flops()

    def _flops(self):
        e = ENC
        T, E, MLP, hd = e["GRID"] ** 2, e["E"], e["MLP"], e["E"] // e["HEADS"]
        lin = 2.0 * T * E * (3 * E + E + 2 * MLP)
        att_w = 4.0 * T * (e["WINDOW"] ** 2) * E          # QK^T and PV over each token's window
        att_g = 4.0 * T * T * E
        kp = -(-3 * e["PATCH"] ** 2 // 128) * 128
        return (2.0 * T * E * 3 * kp + sum(lin + (att_g if i in e["GLOBAL"] else att_w) for i in range(e["DEPTH"]))
                + neck_flops(e["GRID"], E, e["NECK_MID"], e["NECK_DIM"]))

    def free(self):
        """Releases the device buffers (weights, tables, activations, levels)."""
        for b in self.keep + [self.image, self.x] + [lv for lv in self.levels if lv is not None]:
            b.free()
        self.prefix.free()
        self.neck.free()
        self.keep, self.levels = [], []

    def forward(self, neck=True):
        self.prefix.forward(self.image, self.x)
        for d in self.blocks:
            self.sh.check(self.sh.lib().samhip_vit_block(self.ctx.handle, self.ctypes.byref(d), self.x.ptr))
        if neck:
            self.neck.forward(self.x, self.levels)

    def host_block(self, i):
        """Block i's weights as numpy arrays (device bytes downloaded) for the oracle."""
        d, sh, ctx = self.blocks[i], self.sh, self.ctx
        e = ENC
        E, MLP = e["E"], e["MLP"]
        out = {}

        class At:
            def __init__(self, ptr):
                self.ptr = ptr

        def get(ptr, n):
            return ctx.download(At(ptr), (n,), np.float32)
        for n, sz in (("norm1_w", E), ("norm1_b", E), ("norm2_w", E), ("norm2_b", E), ("qkv_b", 3 * E),
                      ("proj_b", E), ("fc1_b", MLP), ("fc2_b", E)):
            out[n] = get(getattr(d, n), sz)
        for n in ("qkv", "proj", "fc1", "fc2"):
            t = getattr(d, n + "_w")
            rows, rb = t.ne[1], sh.row_bytes(t.type, t.ne[0])
            out[n + "_type"] = t.type
            out[n + "_w"] = ctx.download(At(t.data), (rows, rb), np.uint8)
        glob = i in e["GLOBAL"]
        n_tok = e["GRID"] ** 2 if glob else e["WINDOW"] ** 2
        out["freqs"] = ctx.download(At(d.freqs_cis), (n_tok, E // e["HEADS"] // 2, 2), np.float32)
        return out


def encoder_roofline(breakdown):
    """Roofline of the encode's two MFMA-bound parts, from the per-image
    kernel times of the events pass (`kernel_ms_per_image`):
      linears: 2*M*N*K of the 32 blocks' qkv, proj, fc1 and fc2 products
               divided by their GEMM time plus their preparation launches
               (activation staging + weight decode, with the folded layer
               norm / erf-GELU), against the fp16 dense peak;
      attention: 4*N_keys*hd flops per query and head (QK^T and PV) over
               each token's window (28 windowed blocks, 576 keys) or the
               whole grid (4 global blocks, 5184 keys) divided by the
               attention launches' time; at F32-accurate operands the MFMA
               issues 3x that work (hi*hi + lo*hi + hi*lo), reported beside
               it as `mfma_frac`."""
    e = ENC
    T, E, MLP = e["GRID"] ** 2, e["E"], e["MLP"]
    n_glob = len(e["GLOBAL"])
    lin_flops = e["DEPTH"] * 2.0 * T * E * (3 * E + E + 2 * MLP)
    lin_names = ("vit_qkv", "vit_proj", "vit_fc1", "vit_fc2")
    lin_ms = sum(v for k, v in breakdown.items() if k in lin_names or k.startswith("stage_"))
    gemm_ms = sum(v for k, v in breakdown.items() if k in lin_names)
    att_flops = ((e["DEPTH"] - n_glob) * 4.0 * T * e["WINDOW"] ** 2 * E + n_glob * 4.0 * T * T * E)
    att_ms = breakdown.get("vit_attention", 0.0)
    lin_ach = lin_flops / (lin_ms * 1e-3) / 1e12 if lin_ms else None
    att_ach = att_flops / (att_ms * 1e-3) / 1e12 if att_ms else None
    return {"bound": "mfma", "achieved": round(lin_ach, 2) if lin_ach else None, "peak": PEAK_FP16_TFLOPS,
            "unit": "TFLOP/s", "frac": round(lin_ach / PEAK_FP16_TFLOPS, 4) if lin_ach else None, "traffic": None,
            "kernel": "ViT linears: qkv/proj/fc1/fc2 GEMMs + their preparation launches (events, per image)",
            "flops_per_image": lin_flops, "ms_per_image": round(lin_ms, 4),
            "gemm_only": {"ms_per_image": round(gemm_ms, 4),
                          "achieved": round(lin_flops / (gemm_ms * 1e-3) / 1e12, 2) if gemm_ms else None},
            "attention": {"bound": "mfma", "achieved": round(att_ach, 2) if att_ach else None,
                          "peak": PEAK_FP16_TFLOPS, "unit": "TFLOP/s",
                          "frac": round(att_ach / PEAK_FP16_TFLOPS, 4) if att_ach else None,
                          "mfma_frac": round(3 * att_ach / PEAK_FP16_TFLOPS, 4) if att_ach else None,
                          "flops_per_image": att_flops, "ms_per_image": round(att_ms, 4),
                          "note": "F32-accurate operands: the MFMA runs 3x the algorithmic flops (mfma_frac)"}}


def encoder_cpu_baseline(enc, seconds_cap=60.0):
    """The oracle's restatement of the same encoder (native quantized
    linears, exact softmax attention) on the host cores, on a bounded
    sample: the prefix, one windowed and one global block, extrapolated to
    the 28 windowed + 4 global blocks of one image."""
    sys.path.insert(0, ROOT)
    from oracle import oracle as O
    O.lib()
    threads = O.max_threads()
    e = ENC
    G, E = e["GRID"], e["E"]
    x = np.random.default_rng(5).standard_normal((G * G, E)).astype(np.float32)
    times = {}
    for label, i in (("windowed", 0), ("global", e["GLOBAL"][0])):
        w = enc.host_block(i)
        t0 = time.perf_counter()
        O.vit_block(w, x, G, G, E, e["HEADS"], e["MLP"], 0 if i in e["GLOBAL"] else e["WINDOW"], O.ROUND_X86, threads)
        times[label] = time.perf_counter() - t0
        if sum(times.values()) > seconds_cap:
            break
    rng = np.random.default_rng(6)
    img = rng.standard_normal((3, e["IMG"], e["IMG"])).astype(np.float32)
    t0 = time.perf_counter()
    O.vit_prefix(img, e["PATCH"], rng.standard_normal((E, 3, e["PATCH"], e["PATCH"])).astype(np.float32) * 0.02,
                 rng.standard_normal((e["POS_GRID"], e["POS_GRID"], E)).astype(np.float32) * 0.1, e["POS_GRID"],
                 np.ones(E, np.float32), np.zeros(E, np.float32), E, threads)
    times["prefix"] = time.perf_counter() - t0
    # the neck on a 24 x 24 crop of the 72 x 72 map (every level's cost is
    # proportional to its pixels), scaled by 9
    crop = x.reshape(G, G, E)[:24, :24].reshape(-1, E)
    t0 = time.perf_counter()
    O.neck(enc.neck_host, crop, 24, E, e["NECK_MID"], e["NECK_DIM"], threads, levels=(0, 1, 2))
    times["neck"] = (time.perf_counter() - t0) * (G / 24) ** 2
    n_glob = len(e["GLOBAL"])
    per_image = (times["prefix"] + (e["DEPTH"] - n_glob) * times["windowed"]
                 + n_glob * times.get("global", times["windowed"]) + times["neck"])
    return {"value": round(per_image * 1e3, 1), "unit": "ms/image", "cores": threads, "kind": "port",
            "sample": f"prefix {times['prefix']:.2f} s + one windowed block {times['windowed']:.2f} s + one global "
                      f"block {times.get('global', float('nan')):.2f} s, extrapolated to 28 windowed + 4 global "
                      f"blocks, + neck levels 0-2 on a 24x24 crop x 9 ({times['neck']:.2f} s); "
                      f"oracle/vit_oracle.c (native Q8 linears, exact-softmax attention, F32 convolutions), OpenMP"}


def encoder_measure(sh, ctx, enc, warmup, iters, fp16_attention=True):
    """ms/image of the image encode (prefix + 32 blocks + neck levels 0-2,
    as the reference's image path runs it, F32-accurate attention), its
    kernel breakdown, ms/image of the ViT alone (prefix + 32 blocks) and,
    with `fp16_attention`, of the encode with fp16 attention operands."""
    for _ in range(warmup):
        enc.forward()
    ctx.synchronize()
    ctx.trace_begin()
    enc.forward()
    prof = ctx.trace_end(capacity=1 << 12)
    t0 = time.perf_counter()
    for _ in range(iters):
        enc.forward()
    ctx.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / iters
    t0 = time.perf_counter()
    for _ in range(iters):
        enc.forward(neck=False)
    ctx.synchronize()
    enc.vit_ms = (time.perf_counter() - t0) * 1e3 / iters
    enc.fp16_attention_ms = None
    if not fp16_attention:
        return ms, prof, kernel_breakdown(prof)
    # the same encode with fp16 attention operands (attention_type F16)
    for d in enc.blocks:
        d.attention_type = sh.F16
    enc.forward()
    ctx.synchronize()
    t0 = time.perf_counter()
    for _ in range(iters):
        enc.forward()
    ctx.synchronize()
    enc.fp16_attention_ms = (time.perf_counter() - t0) * 1e3 / iters
    for d in enc.blocks:
        d.attention_type = sh.F32
    return ms, prof, kernel_breakdown(prof)


def kernel_breakdown(prof):
    """Per-image ms by launch name from one traced forward."""
    by = {}
    for name, wt, m, n, k, kms in prof:
        # attention launches carry their key-split count (vit_attention_splitS)
        by.setdefault("vit_attention" if name.startswith("vit_attention") else name, []).append((m, n, k, kms))
    return {name: round(sum(r[3] for r in rs), 4) for name, rs in sorted(by.items(), key=lambda t: -sum(r[3] for r in t[1]))}


def encoder_workload(args, sh, ctx):
    """--workload encoder: the full vision encoder forward, ms/image."""
    qt = {"q4_k": sh.Q4_K, "q5_k": sh.Q5_K, "q6_k": sh.Q6_K, "q8_0": sh.Q8_0}[args.format]
    log("building the vision encoder")
    enc = Encoder(sh, ctx, qt)
    ms, prof, breakdown = encoder_measure(sh, ctx, enc, args.warmup, args.steps)
    # the single fc1 launch of a block, beside the encode's roofline
    fc1 = [r for r in prof if r[0] == "vit_fc1"]
    m_, n_, k_ = fc1[0][2], fc1[0][3], fc1[0][4]
    fc1_ms = float(np.mean([r[5] for r in fc1]))
    ach = 2.0 * m_ * n_ * k_ / (fc1_ms * 1e-3) / 1e12
    roof = encoder_roofline(breakdown)
    roof["fc1_launch"] = {"achieved": round(ach, 2), "frac": round(ach / PEAK_FP16_TFLOPS, 4),
                          "kernel": "vit_fc1 (fp16 GEMM + bias + GELU)", "shape": {"M": m_, "N": n_, "K": k_},
                          "launch_ms": round(fc1_ms, 5)}
    result = {
        "metric": "SAM3 vision encode ms/image @1008px", "value": round(ms, 3), "unit": "ms/image", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 3), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp16", "data": "synthetic",
        "config": {"workload": f"SAM 3 vision encoder forward, 1008x1008x3 image, 72x72 tokens, width 1024, 32 blocks "
                               f"(window 24, global 7/15/23/31), 16 heads, MLP 4736; {sh.TYPE_NAMES[qt]} qkv/proj/fc1, "
                               f"q8_0 fc2; SimpleFPN neck levels 0-2 (F32 columns); random-init weights", "batch": 1,
                   "parallelism": "single-gpu"},
        "tflops_effective": round(enc.flops / (ms * 1e-3) / 1e12, 2),
        "vit_ms_per_image": round(enc.vit_ms, 3),
        "fp16_attention_ms_per_image": round(enc.fp16_attention_ms, 3),
        "roofline": roof,
        "kernel_ms_per_image": breakdown,
        "device": ctx.query().device_name.decode(),
    }
    if not args.no_cpu_baseline:
        log("timing the encoder CPU baseline")
        result["cpu_baseline"] = encoder_cpu_baseline(enc)
    else:
        result["cpu_baseline"] = None
    return result


def linear_set(sh, ctx, m, items, steps, warmup, seed=0, rotate=1):
    """Times a set of tall products [(label, weight type, K, N)] at M = m,
    each with its own X and Y, weights N(0, 0.02^2) and X N(0, 1): whole-step
    TOPS (activation staging, weight decode and GEMM), per-product event
    times, and the dominant kernel's roofline (events on its launch stream).
    `rotate` > 1 gives every product that many independent W / X / Y sets,
    step i running set i % rotate, so that a set whose bytes fit the 256 MB
    MALL is not served from it on the next step."""
    rng = np.random.default_rng(seed + 1)
    sets = []
    for r in range(rotate):
        ops = []
        for label, qt, k, n in items:
            wf = ctx.upload((np.random.default_rng(seed + 7 * r).standard_normal((n, k)) * 0.02).astype(np.float32))
            wq = ctx.alloc(n * sh.row_bytes(qt, k))
            ctx.quantize_rows(qt, wf.ptr, 4 * k, wq.ptr, n, k, sh.ROUND_REF)
            ctx.synchronize()
            wf.free()
            xb = ctx.upload(rng.standard_normal((m, k)).astype(np.float32))
            yb = ctx.alloc(m * n * 4)
            ops.append((label, qt, k, n, sh.tensor(qt, k, n, wq.ptr), sh.tensor(sh.F32, k, m, xb.ptr),
                        sh.tensor(sh.F32, n, m, yb.ptr), [wq, xb, yb]))
        sets.append(ops)
    ops = sets[0]

    def step(i=0):
        for _, _, _, _, w, x, y, _ in sets[i % rotate]:
            ctx.mul_mat(w, x, y)

    for i in range(warmup):
        step(i)
    ctx.trace_begin()
    for r in range(rotate):
        step(warmup + r)
    prof = ctx.trace_end(capacity=4 * len(ops) * rotate + 16)
    ctx.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step(i)
    ctx.synchronize()
    elapsed = time.perf_counter() - t0
    flops = sum(2.0 * m * n * k for _, _, k, n, *_ in ops)
    per_kernel = collections.defaultdict(float)
    for r in prof:
        per_kernel[r[0]] += r[5]
    dom = max(per_kernel, key=per_kernel.get)
    recs = [r for r in prof if r[0] == dom]
    shape = max({(r[2], r[3], r[4]) for r in recs}, key=lambda sh_: sum(r[5] for r in recs if (r[2], r[3], r[4]) == sh_))
    sel = [r for r in recs if (r[2], r[3], r[4]) == shape]
    ms = float(np.mean([r[5] for r in sel]))
    mm, nn, kk = shape
    qt = sel[0][1]
    ach = 2.0 * mm * nn * kk / (ms * 1e-3) / 1e12
    alg_bytes = nn * sh.row_bytes(qt, kk) + mm * kk * 4 + mm * nn * 4
    products = []
    for label, qt_, k, n, *_ in ops:
        t = sum(r[5] for r in prof if r[1] == qt_ and r[3] == n and r[4] == k) / rotate
        products.append({"product": label, "M": m, "N": n, "K": k, "ms": round(t, 5),
                         "tops": round(2.0 * m * n * k / (t * 1e-3) / 1e12, 2) if t else None})
    set_bytes = sum(n * sh.row_bytes(qt_, k) + m * k * 4 + m * n * 4 for _, qt_, k, n, *_ in ops)
    for st in sets:
        for o in st:
            for b in o[7]:
                b.free()
    return {"value": round(flops * steps / elapsed / 1e12, 3), "unit": "TOPS",
            "ms_per_step": round(elapsed * 1e3 / steps, 4), "steps": steps, "warmup": warmup,
            "rotation": {"sets": rotate, "bytes_per_set": set_bytes, "bytes_rotated": set_bytes * rotate},
            "pct_int8_peak": round(100 * flops * steps / elapsed / 1e12 / PEAK_INT8_TOPS, 2),
            "products": products,
            "roofline": {"bound": "mfma", "achieved": round(ach, 2), "peak": PEAK_FP16_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(ach / PEAK_FP16_TFLOPS, 4), "traffic": hbm_traffic(dom, shape), "kernel": dom,
                         "weight_type": sh.TYPE_NAMES.get(qt, str(qt)), "shape": {"M": mm, "N": nn, "K": kk},
                         "launch_ms": round(ms, 5), "launches": len(sel),
                         "hbm_gbps_algorithmic": round(alg_bytes / (ms * 1e-3) / 1e9, 1)}}


def other_configs(args, sh, ctx, ops, xbuf):
    """The workload's other configurations, each measured in this run with
    its own roofline: (1) the single Q8_0 ViT fc1 linear, (3) the text and
    fusion/decoder linear streams (Q8_0 and Q4_K each), (5) the batch of 8
    images with mixed per-module formats (vision qkv/proj Q6_K, fc1 Q5_K, fc2
    Q8_0 at M = 41,472; its text/fusion/decoder linears are Q8_0, the streams
    of (3))."""
    out = {}
    log("config 1: single Q8_0 fc1")
    out["1_single_q8_0_fc1"] = {"workload": "ViT fc1 1024->4736, Q8_0 weights, M=5184; 3 W/X/Y sets rotated "
                                            "(374 MB, past the 256 MB MALL)",
                                **linear_set(sh, ctx, M_TOKENS, [("fc1:q8_0", sh.Q8_0, 1024, 4736)],
                                             args.steps, args.warmup, rotate=3)}
    sub = argparse.Namespace(**vars(args))
    sub.cpu_seconds = min(args.cpu_seconds, 5.0)
    sub.steps = max(args.steps, 10)
    for fmt in ("q8_0", "q4_k"):
        log(f"config 3: text stream {fmt}")
        r = text_stream(sub, sh, ctx, fmt)
        out[f"3_text_stream_{fmt}"] = {k: r[k] for k in ("metric", "value", "unit", "ms_per_step", "roofline",
                                                           "eager_ms_per_step", "kernel_ms_per_step", "cpu_baseline")}
    for fmt in ("q8_0", "q4_k"):
        log(f"config 3: fusion/decoder stream {fmt}")
        r = detector_stream(sub, sh, ctx, fmt)
        out[f"3_detector_stream_{fmt}"] = {k: r[k] for k in ("metric", "value", "unit", "ms_per_step", "tops",
                                                               "roofline", "cpu_baseline")}
    log("config 5: batch of 8 images, mixed formats")
    m8 = 8 * M_TOKENS
    out["5_batch8_mixed"] = {"workload": "8 images (M=41472): qkv 1024->3072 and proj 1024->1024 Q6_K, fc1 "
                                         "1024->4736 Q5_K, fc2 4736->1024 Q8_0; 4 mul_mat per step",
                             **linear_set(sh, ctx, m8, [("qkv:q6_K", sh.Q6_K, 1024, 3072),
                                                        ("proj:q6_K", sh.Q6_K, 1024, 1024),
                                                        ("fc1:q5_K", sh.Q5_K, 1024, 4736),
                                                        ("fc2:q8_0", sh.Q8_0, 4736, 1024)],
                                          max(3, args.steps // 4), 2)}
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--compute", choices=["native", "f16"], default="native")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU time budget of the stream baselines")
    ap.add_argument("--cpu-rows", type=int, default=64)
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the other configurations' lines (single Q8_0 fc1, text and fusion/decoder streams, "
                         "batch-8 mixed formats) of the headline run")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--trace", choices=["dominant", "all", "none"], default="dominant",
                    help="launches bracketed by HIP events inside the timed region")
    ap.add_argument("--trace-every", type=int, default=5,
                    help="bracket the traced launches of every N-th timed step only (1: every step)")
    ap.add_argument("--workload", choices=["vit", "text", "encoder", "detector", "linear"], default="vit",
                    help="vit: the ViT linear sweep (headline, with the encoder's ms/image beside it); text: the "
                         "M=32 text-encoder linear stream; encoder: the vision encoder forward alone; linear: the "
                         "four ViT linears at M=5184 in one weight format (--format, default q8_0), 3 rotated "
                         "W/X/Y sets")
    ap.add_argument("--format", choices=["q8_0", "q4_k", "q5_k", "q6_k"], default=None,
                    help="weight format of the text stream (default q8_0) or of the encoder's K-quant linears "
                         "(default q4_k)")
    ap.add_argument("--no-encoder", action="store_true", help="skip the vision-encoder measurement of the headline run")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only the plain copy used to scale HBM traffic counters")
    ap.add_argument("--blas-calibration", action="store_true",
                    help="time hipBLASLt (torch.mm, fp16 operands, F32 output) at the four ViT shapes and exit")
    ap.add_argument("--summarize-profiles", metavar="DIR",
                    help="write profiles/ summaries from rocprofv3 CSV output in DIR and exit")
    args = ap.parse_args()
    if args.copy_calibration:
        copy_calibration()
        return
    if args.blas_calibration:
        blas_calibration()
        return
    if args.summarize_profiles:
        summarize_profiles(args.summarize_profiles, PROFILE_COMMANDS)
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE {world}); the per-GPU shard is the single-GPU run.", file=sys.stderr)
        sys.exit(2)

    sh = load_samhip()
    compute = sh.COMPUTE_Q8_NATIVE if args.compute == "native" else sh.COMPUTE_F16
    ctx = sh.Context(0, compute, sh.ROUND_X86)
    if args.workload == "text":
        result = text_stream(args, sh, ctx, args.format or "q8_0")
        ctx.close()
        print(json.dumps(result), flush=True)
        return
    if args.workload == "detector":
        result = detector_stream(args, sh, ctx, args.format or "q8_0")
        ctx.close()
        print(json.dumps(result), flush=True)
        return
    if args.workload == "encoder":
        args.format = args.format or "q4_k"
        result = encoder_workload(args, sh, ctx)
        ctx.close()
        print(json.dumps(result), flush=True)
        return
    if args.workload == "linear":
        fmt = args.format or "q8_0"
        qt = {"q4_k": sh.Q4_K, "q5_k": sh.Q5_K, "q6_k": sh.Q6_K, "q8_0": sh.Q8_0}[fmt]
        items = [(f"{name}:{fmt}", qt if k % 256 == 0 or qt == sh.Q8_0 else sh.Q8_0, k, n) for name, k, n in SHAPES]
        r = linear_set(sh, ctx, M_TOKENS, items, args.steps, args.warmup, rotate=3)
        result = {"metric": f"ViT linears at M={M_TOKENS}, {fmt} (fc2 Q8_0), TOPS", "value": r["value"], "unit": "TOPS",
                  "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": r["ms_per_step"],
                  "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
                  "data": "synthetic", "config": {"workload": f"qkv, proj, fc1, fc2 at M={M_TOKENS}, 3 rotated sets",
                                                   "tall_int8": os.environ.get("SAMHIP_TALL_INT8", "0")},
                  "roofline": r["roofline"], "products": r["products"], "rotation": r["rotation"],
                  "device": ctx.query().device_name.decode()}
        ctx.close()
        print(json.dumps(result), flush=True)
        return
    plan = products(sh)

    log("preparing inputs")
    # every product reads its own activation rows and writes its own output,
    # so one step touches 1.1 GB (past the 256 MB MALL) as a forward would
    rng = np.random.default_rng(1)
    xrows = {k: rng.standard_normal((M_TOKENS, k)).astype(np.float32) for k in sorted({p[2] for p in plan})}
    xbuf = []     # one buffer per product (labels repeat: fc2 is Q8_0 in every profile)
    ops = []
    for label, qt, k, n in plan:
        xbuf.append(ctx.upload(xrows[k]))
        wf = ctx.upload((np.random.default_rng(0).standard_normal((n, k)) * 0.02).astype(np.float32))
        wq = ctx.alloc(n * sh.row_bytes(qt, k))
        ctx.quantize_rows(qt, wf.ptr, 4 * k, wq.ptr, n, k, sh.ROUND_REF)
        ctx.synchronize()
        wf.free()
        yb = ctx.alloc(M_TOKENS * n * 4)
        w = sh.tensor(qt, k, n, wq.ptr)
        x = sh.tensor(sh.F32, k, M_TOKENS, xbuf[-1].ptr)
        y = sh.tensor(sh.F32, n, M_TOKENS, yb.ptr)
        if not sh.lib().samhip_supports_mul_mat(w, x, y):
            raise RuntimeError(f"unsupported product {label}")
        ops.append((label, qt, k, n, w, x, y, wq, yb))
    del xrows

    def step():
        for _, _, _, _, w, x, y, _, _ in ops:
            ctx.mul_mat(w, x, y)

    for _ in range(args.warmup):
        step()
    ctx.synchronize()
    log(f"warmup done ({args.warmup} steps)")

    # untimed profiling pass: every launch bracketed by events, for the
    # per-product breakdown and to name the dominant kernel
    prof_steps = max(1, min(args.steps, 5))
    ctx.trace_begin()
    for _ in range(prof_steps):
        step()
    prof = ctx.trace_end(capacity=4 * len(ops) * prof_steps + 16)
    by_kernel = {}
    for name, wt, m, n, k, ms in prof:
        by_kernel.setdefault(name, []).append((wt, m, n, k, ms))
    total = {name: sum(r[4] for r in rs) for name, rs in by_kernel.items()}
    dominant = max(total, key=total.get)

    def mean_ms(recs, qt, n, k, prefix):
        sel = [r[5] for r in recs if r[1] == qt and r[3] == n and r[4] == k and r[0].startswith(prefix)]
        return float(np.mean(sel)) if sel else 0.0

    per_product = []
    for label, qt, k, n, *_ in ops:
        g = mean_ms(prof, qt, n, k, "gemm")
        s = mean_ms(prof, qt, n, k, "stage")
        d = mean_ms(prof, qt, n, k, "dequant")
        per_product.append({"product": label, "M": M_TOKENS, "N": n, "K": k, "gemm_ms": round(g, 5),
                            "stage_ms": round(s, 5), "dequant_ms": round(d, 5),
                            "gemm_tflops": round(2.0 * M_TOKENS * n * k / g / 1e9, 2) if g else None,
                            "linear_tops": round(2.0 * M_TOKENS * n * k / (g + s + d) / 1e9, 2) if g else None})
    kernel_share = {name: round(v / sum(total.values()), 4) for name, v in sorted(total.items(), key=lambda t: -t[1])}

    # timed region: events around the dominant kernel's launches (or none /
    # all) in every trace_every-th step; each bracket adds two event records
    # (several microseconds of GPU time), so the other steps run without
    every = max(1, args.trace_every)
    log(f"timing {args.steps} steps (trace: {args.trace} in every {every}. step, dominant kernel {dominant})")
    ctx.synchronize()
    if args.trace != "none":
        ctx.trace_begin(dominant if args.trace == "dominant" else None)
        ctx.trace_pause(every > 1)
    t0 = time.perf_counter()
    for i in range(args.steps):
        if args.trace != "none" and every > 1 and i % every == every - 1:
            ctx.trace_pause(False)
            step()
            ctx.trace_pause(True)
        else:
            step()
    if args.trace != "none":
        records = ctx.trace_end(capacity=4 * len(ops) * args.steps + 16)   # waits for the stream
    else:
        ctx.synchronize()
        records = []
    elapsed = time.perf_counter() - t0
    log(f"timed {args.steps} steps in {elapsed * 1e3:.1f} ms")

    flops_step = sum(2.0 * M_TOKENS * n * k for _, _, k, n, *_ in ops)
    ms_step = elapsed * 1e3 / args.steps
    tops = flops_step * args.steps / elapsed / 1e12

    # roofline of the dominant kernel from the HIP events on its launch stream
    # (timed region when traced there, else the profiling pass)
    launches = [r for r in (records or prof) if r[0] == dominant]
    shapes = {(r[2], r[3], r[4]) for r in launches}
    m_, n_, k_ = max(shapes, key=lambda sh_: sum(r[5] for r in launches if (r[2], r[3], r[4]) == sh_))
    same = [r[5] for r in launches if (r[2], r[3], r[4]) == (m_, n_, k_)]
    avg_ms = float(np.mean(same))
    qt_dom = collections.Counter(r[1] for r in launches if (r[2], r[3], r[4]) == (m_, n_, k_)).most_common(1)[0][0]
    flops = 2.0 * m_ * n_ * k_
    achieved = flops / (avg_ms * 1e-3) / 1e12
    alg_bytes = n_ * k_ * 2 + m_ * k_ * 2 + m_ * n_ * 4
    roofline = {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_FP16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_FP16_TFLOPS, 4), "traffic": hbm_traffic(dominant, (m_, n_, k_)),
                "kernel": dominant, "weight_type": sh.TYPE_NAMES.get(qt_dom, str(qt_dom)),
                "shape": {"M": m_, "N": n_, "K": k_}, "launch_ms": round(avg_ms, 5),
                "launches": len(same),
                "events_in": (f"timed region, every {every}. step" if every > 1 else "timed region") if records
                else "profiling pass",
                "flops_per_launch": flops, "algorithmic_bytes_per_launch": int(alg_bytes),
                "hbm_gbps_algorithmic": round(alg_bytes / (avg_ms * 1e-3) / 1e9, 1),
                "pct_int8_peak": round(100 * achieved / PEAK_INT8_TOPS, 2)}

    result = {
        "metric": METRIC, "value": round(tops, 3), "unit": "TOPS", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp16", "data": "synthetic",
        "config": {"workload": "SAM 3 ViT K-quant linear sweep (Q4_K/Q5_K/Q6_K qkv, proj, fc1; fc2 Q8_0) at "
                               "M=5184 tokens, 12 mul_mat per step",
                   "m_tokens": M_TOKENS,
                   "compute": ("Q8_0/Q8_K activation codes (bit-exact ggml packing) x fp16(to_float(W)) on fp16 "
                               "MFMA, F32 accumulation" if compute == sh.COMPUTE_Q8_NATIVE
                               else "fp16(X) x fp16(to_float(W)) on fp16 MFMA, F32 accumulation"),
                   "parallelism": "single-gpu", "activation": "F32 in HBM, one buffer per product",
                   "output": "F32, one buffer per product"},
        "pct_int8_peak": round(100 * tops / PEAK_INT8_TOPS, 2),
        "roofline": roofline,
        "products": per_product,
        "kernel_time_share": kernel_share,
        "device": ctx.query().device_name.decode(),
    }
    enc = None
    if not args.no_encoder:
        # the metric's second figure: the Q4_K vision encoder forward, measured
        # after the sweep's timed region (its own warmup and timing)
        for b in [o[7] for o in ops] + [o[8] for o in ops] + xbuf:
            b.free()
        ops, xbuf = [], []
        log("building the Q4_K vision encoder")
        enc = Encoder(sh, ctx, sh.Q4_K)
        enc_ms, _, breakdown = encoder_measure(sh, ctx, enc, 3, 10)
        result["vision_encoder"] = {
            "ms_per_image": round(enc_ms, 3), "images_per_s": round(1e3 / enc_ms, 2),
            "vit_ms_per_image": round(enc.vit_ms, 3),
            "fp16_attention_ms_per_image": round(enc.fp16_attention_ms, 3),
            "tflops_effective": round(enc.flops / (enc_ms * 1e-3) / 1e12, 2),
            "config": "1008x1008x3 image, 72x72 tokens, width 1024, 32 blocks (window 24, global 7/15/23/31), "
                      "16 heads, MLP 4736; Q4_K qkv/proj/fc1, Q8_0 fc2; SimpleFPN neck levels 0-2 (F32 columns); "
                      "random-init weights; batch 1; 3 warmup + 10 timed forwards",
            "roofline": encoder_roofline(breakdown),
            "kernel_ms_per_image": breakdown}
        # the Q8_0 variant: every linear Q8_0 (472 MB of packed weights)
        log("building the Q8_0 vision encoder")
        enc8 = Encoder(sh, ctx, sh.Q8_0, seed=3)
        ms8, _, bd8 = encoder_measure(sh, ctx, enc8, 3, 10, fp16_attention=False)
        result["vision_encoder"]["q8_0_variant"] = {
            "ms_per_image": round(ms8, 3), "images_per_s": round(1e3 / ms8, 2),
            "vit_ms_per_image": round(enc8.vit_ms, 3),
            "tflops_effective": round(enc8.flops / (ms8 * 1e-3) / 1e12, 2),
            "config": "as above with every linear (qkv/proj/fc1/fc2) Q8_0; 3 warmup + 10 timed forwards",
            "roofline": encoder_roofline(bd8), "kernel_ms_per_image": bd8}
        enc8.free()
    if not args.no_configs:
        result["configs"] = other_configs(args, sh, ctx, ops, xbuf)
    if not args.no_cpu_baseline:
        log("timing the CPU baseline")
        result["cpu_baseline"] = cpu_baseline(plan, args.cpu_rows)
        if enc is not None:
            log("timing the encoder CPU baseline")
            result["vision_encoder"]["cpu_baseline"] = encoder_cpu_baseline(enc)
    else:
        result["cpu_baseline"] = None
    ctx.close()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
