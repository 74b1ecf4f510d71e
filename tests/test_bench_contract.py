"""CPU checks of bench.py's contract and workload plans (no GPU needed)."""
import collections
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout.strip() == ""


def test_detector_plan_matches_the_reference_layers():
    """6 fusion layers x 10 products and 6 decoder layers x 14
    (src/models/sam3/fusion_encoder.hpp:46-145, src/models/sam3/detector.hpp:343-479);
    q/k/v are row-offset views inside their fused [3D, D] in-projection."""
    plan = bench.detector_plan()
    assert len(plan) == 6 * 10 + 6 * 14
    d, f = bench.DET_D, bench.DET_FFN
    for label, key, rows, off, n, k, (src, xk) in plan:
        assert 0 <= off and off + n <= rows and xk == k and src in bench.DET_M
        if key.endswith("_in"):
            assert rows == 3 * d and off in (0, d, 2 * d)
        assert (n, k) in ((d, d), (f, d), (d, f))
    shapes = collections.Counter((bench.DET_M[p[6][0]], p[4], p[5]) for p in plan)
    assert shapes[(5184, d, d)] == 6 * 6 + 6 * 2      # fusion q,k,v,sa_out,ca_q,ca_out + decoder image k,v
    assert shapes[(201, d, d)] == 6 * 8               # decoder sa q,k,v,out + two cross-attention q,out
    assert shapes[(33, d, d)] == 6 * 2 + 6 * 2        # prompt / text k,v


def test_text_stream_shapes():
    assert [s[1:] for s in bench.TEXT_SHAPES] == [(1024, 3072), (1024, 1024), (1024, 4096), (4096, 1024)]
    assert bench.TEXT_LAYERS == 24 and bench.TEXT_M == 32


def test_cpu_baseline_protocol_on_a_small_plan():
    """Both CPU paths at all threads and at 4, AB/BA-alternated samples with
    median and P95, and the host's CPU model and ISA flags."""
    plan = [("a:q8_0", 8, 64, 32), ("b:q4_K", 12, 256, 16)]
    r = bench.cpu_baseline(plan, rows=4, samples=3, warmup=1)
    assert r["kind"] == "port" and r["unit"] == "TOPS" and r["value"] > 0 and r["cores"] >= 1
    threads = {p["threads"] for p in r["paths"].values()}
    assert min(4, r["cores"]) in threads and r["cores"] in threads
    for name, p in r["paths"].items():
        assert name.split("_")[0] in ("native", "decode")
        assert p["samples"] == 3 and 0 < p["median_ms"] <= p["p95_ms"]
    assert "model" in r["host"] and isinstance(r["host"]["isa"], list)
