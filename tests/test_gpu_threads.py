"""The boundary's threading contract (include/samhip.h): a context is
single-threaded and stream-ordered, distinct contexts may be used from
distinct host threads at the same time.  The reference serializes a model
behind one execution mutex and names independent contexts as the way to run
concurrently (src/models/sam3/state.hpp:19-22).

Two host threads, each with its own context, run interleaved mul_mat
(tall, fused-skinny and strip-skinny products) and get_rows calls at the same
time; every result must be bit-identical to the same calls run serially on
one context.  ctypes releases the GIL around each library call, so the
threads are inside the library concurrently."""

import sys
import threading

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROUNDS = 6


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _workload(oracle, seed):
    rng = np.random.default_rng(seed)
    jobs = []
    for qtype, (m, n, k) in ((oracle.Q4_K, (512, 384, 1024)), (oracle.Q8_0, (32, 1024, 1024)),
                             (oracle.Q6_K, (201, 256, 256)), (oracle.Q8_0, (300, 256, 2048))):
        w = oracle.quantize(qtype, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
        x = rng.standard_normal((m, k)).astype(np.float32)
        jobs.append(("mul_mat", qtype, w, x))
    table = rng.standard_normal((300, 256)).astype(np.float32)
    ids = rng.integers(0, 300, 32).astype(np.int32)
    jobs.append(("get_rows", table, ids))
    return jobs


def _run(samhip, ctx, jobs):
    out = []
    for _ in range(ROUNDS):
        for job in jobs:
            if job[0] == "mul_mat":
                _, qtype, w, x = job
                out.append(ctx.matmul(qtype, w, x))
            else:
                _, table, ids = job
                k = table.shape[1]
                src, idb, dst = ctx.upload(table), ctx.upload(ids), ctx.alloc(len(ids) * k * 4)
                ctx.get_rows(samhip.tensor(samhip.F32, k, table.shape[0], src.ptr),
                             samhip.tensor(samhip.I32, len(ids), 1, idb.ptr),
                             samhip.tensor(samhip.F32, k, len(ids), dst.ptr))
                out.append(ctx.download(dst, (len(ids), k), np.float32))
    return out


def test_two_contexts_on_two_threads_match_serial(samhip, oracle):
    jobs = [_workload(oracle, 1), _workload(oracle, 2)]
    say("case threads: serial reference")
    with samhip.Context(0, samhip.COMPUTE_Q8_NATIVE, samhip.ROUND_X86) as ctx:
        serial = [_run(samhip, ctx, j) for j in jobs]
    say("case threads: two contexts, two threads")
    results, errors = [None, None], []
    start = threading.Barrier(2)

    def worker(i):
        try:
            with samhip.Context(0, samhip.COMPUTE_Q8_NATIVE, samhip.ROUND_X86) as ctx:
                start.wait(timeout=60)
                results[i] = _run(samhip, ctx, jobs[i])
        except Exception as e:   # reported below, with the thread's index
            errors.append((i, repr(e)))

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=300)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    assert not errors, errors
    for i in range(2):
        assert len(results[i]) == len(serial[i])
        for a, b in zip(results[i], serial[i]):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
