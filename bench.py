#!/usr/bin/env python3
"""Route benchmark on one MI355X.

Headline workload: MLA latent-centroid route, 1,000,000 nodes x 288 fp32
(unit-norm Gaussian), one query per call, top-3; the bank and the query are
resident in HBM before timing.  Each step is one route call through the C
ABI (kernel + top-k + device->host copy of the k results).  Reported:

* value      p50 wall latency per call (ms) over --steps calls
* roofline   HBM roofline of the route kernel: algorithmic bytes per launch
             (N*D*4 row bytes + N*4 norm bytes) / mean kernel time from HIP
             events recorded on the library's route stream
* gqa        the ragged GQA route (512 nodes, lengths U[16,512], 4 layers x 8
             kv heads x 128, bf16, 32 query heads, top-3): p50/p99 and its
             roofline (sum(L_i) * 32 * 128 * 2 bytes)
* store_route  the store's route law (lexical bonus + route filters) on
             the device, 1M nodes, against the plain route
* payload    packed graft payload unpack on the device: kernel roofline and
             one node mount against host dequant + fp16 upload
* bank_bridge  arena-bridge refresh time at about 1% churn per epoch
             (100k MLA nodes; 512 ragged GQA nodes) against a full rebuild
* cpu_baseline  the oracle's fp64 route law on the same 1M bank, timed on
             this host's cores for a bounded number of queries

Prints one JSON line on stdout; progress goes to stderr.

`roofline.traffic` is the HBM bytes per launch that rocprofv3 counted for
the kernel (FETCH_SIZE + WRITE_SIZE, each scaled by what the counter reads
for a device-to-device copy of known size); the figures and the commands
that produced them are in profiles/, read from profiles/traffic.json.
`--copy-calibration` runs that copy (1 GiB, 5 times) and nothing else.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def pct(xs, p):
    return float(np.percentile(np.asarray(xs, dtype=np.float64), p))


class route_events:
    """Timed routes inside keep HIP events around their kernels on the
    route's stream (GRM_HIP_ROUTE_TIMING=events, read by the library at
    each route); by default a timed route that completes through flags
    takes its device time from the device's constant clock instead.  The
    kernel times behind every roofline figure are taken in here."""

    def __enter__(self):
        self._old = os.environ.get("GRM_HIP_ROUTE_TIMING")
        os.environ["GRM_HIP_ROUTE_TIMING"] = "events"
        return self

    def __exit__(self, *exc):
        if self._old is None:
            os.environ.pop("GRM_HIP_ROUTE_TIMING", None)
        else:
            os.environ["GRM_HIP_ROUTE_TIMING"] = self._old
        return False


def host_cpu() -> dict:
    """What the CPU baselines ran on: core counts and the CPU model."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count()
    return {"nproc": os.cpu_count(), "affinity_cpus": affinity, "model": model,
            "omp_num_threads_env": os.environ.get("OMP_NUM_THREADS")}


def cpu_threads_all() -> int:
    """Every host thread this process may use: the CPUs in its affinity
    mask, or fewer when OMP_NUM_THREADS sets the process's share."""
    info = host_cpu()
    n = int(info["affinity_cpus"] or 1)
    env = info["omp_num_threads_env"]
    if env and env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(1, n)


def time_cpu(fn, seconds: float, *, warmup: int = 4, min_calls: int = 3,
             max_calls: int = 50) -> list[float]:
    """Per-call wall times in ms: `warmup` untimed calls, then calls timed
    with perf_counter_ns until `seconds` have passed (at least `min_calls`,
    at most `max_calls`), as the reference's router baseline harness does
    (scripts/grm_router_baseline.py:348-359, 419-432)."""
    for _ in range(warmup):
        fn()
    times = []
    end = time.perf_counter() + seconds
    while len(times) < min_calls or (time.perf_counter() < end and len(times) < max_calls):
        t0 = time.perf_counter_ns()
        fn()
        times.append((time.perf_counter_ns() - t0) / 1e6)
    return times


def cpu_figure(times: list[float], threads: int) -> dict:
    return {"p50_ms": round(pct(times, 50), 4), "p95_ms": round(pct(times, 95), 4),
            "calls": len(times), "threads": threads}


def copy_calibration(gib: float = 1.0, reps: int = 5) -> dict:
    """A device-to-device copy of known size, for scaling rocprofv3's
    FETCH_SIZE / WRITE_SIZE counters to bytes."""
    import torch

    n = int(gib * (1 << 30)) // 4
    src = torch.full((n,), 1.0, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    return {"copy_bytes_read": n * 4, "copy_bytes_written": n * 4, "reps": reps}


def load_traffic() -> dict:
    path = ROOT / "profiles" / "traffic.json"
    try:
        return json.loads(path.read_text())
    except (OSError, ValueError):
        return {}


def bench_latent_entry(bank, dim: int, k: int, steps: int) -> dict:
    """Route key from a device-resident latent block (512 tokens x dim
    fp16, what a forward pass leaves on the GPU), routed in one call,
    against the host round trip the reference makes: copy the latent
    back, form latent_centroid with numpy (core/kv_graft.py:131-142) and
    route the host query."""
    from graftrepository_amd.payload import DeviceArray

    rng = np.random.default_rng(5)
    lat = rng.standard_normal((512, dim)).astype(np.float16)
    dev_ms, host_ms = [], []
    with DeviceArray.from_host(lat) as d_lat:
        for i in range(steps + 3):
            t0 = time.perf_counter()
            r1 = bank.route_latent(d_lat, 512, k, dtype="f16", timed=False)
            t1 = time.perf_counter()
            back = d_lat.to_host()
            c = back.astype(np.float32).mean(0)
            key = c / (np.linalg.norm(c) + 1e-8)
            r2 = bank.route(key[None], k, timed=False)
            t2 = time.perf_counter()
            if i >= 3:
                dev_ms.append((t1 - t0) * 1e3)
                host_ms.append((t2 - t1) * 1e3)
    same = bool(np.array_equal(r1.ids, r2.ids))
    out = {"latent_tokens": 512, "latent_dtype": "f16",
           "device_key_route_ms_p50": round(pct(dev_ms, 50), 4),
           "host_round_trip_route_ms_p50": round(pct(host_ms, 50), 4),
           "same_ids": same}
    log(f"[mla latent] device key + route {out['device_key_route_ms_p50']:.3f} ms, "
        f"host round trip {out['host_round_trip_route_ms_p50']:.3f} ms, same ids {same}")
    return out


def bench_mla(steps: int, warmup: int):
    from graftrepository_amd import MlaNodeBank, workloads as wl
    from graftrepository_amd.mla_probe import HipProbe

    cfg = wl.MLA_HEADLINE
    n, d, k = cfg["nodes"], cfg["dim"], cfg["topk"]
    t0 = time.time()
    rows = wl.mla_rows(n, d, seed=cfg["seed"])
    q = wl.mla_queries(1, d, seed=cfg["seed"])
    log(f"[mla] generated {n}x{d} bank in {time.time() - t0:.1f}s")
    bank = MlaNodeBank(rows)
    probe = HipProbe()
    dq = probe.upload_queries(q)
    for _ in range(warmup):
        bank.route(dq, k, on_device=True, query_count=1)
    # latency: routes that ask for no device time, as a caller makes them
    # (completion seen through the blocks' flags); kernel time: the same
    # routes with stream events around the kernel
    walls, devs, timed_walls = [], [], []
    for _ in range(steps):
        r = bank.route(dq, k, on_device=True, query_count=1, timed=False)
        walls.append(r.wall_ms)
    ids = r.ids[0].copy()
    scores = r.scores[0].copy()
    # a fixed population of 1000 calls for p50/p99, whatever --steps is
    calls_1000 = []
    for _ in range(1000):
        r = bank.route(dq, k, on_device=True, query_count=1, timed=False)
        calls_1000.append(r.wall_ms)
    assert np.array_equal(r.ids[0], ids) and np.array_equal(r.scores[0], scores)
    with route_events():
        for _ in range(min(steps, 300)):
            r = bank.route(dq, k, on_device=True, query_count=1)
            assert np.array_equal(r.ids[0], ids) and np.array_equal(r.scores[0], scores)
            devs.append(r.device_ms)
    # what a caller that asks for device time waits (device clock, flags)
    for _ in range(min(steps, 300)):
        r = bank.route(dq, k, on_device=True, query_count=1)
        assert np.array_equal(r.ids[0], ids) and np.array_equal(r.scores[0], scores)
        timed_walls.append(r.wall_ms)
    dq.close()
    latent = bench_latent_entry(bank, d, k, max(20, steps // 10))
    bank.close()
    bytes_per_launch = n * d * 4 + n * 4
    mean_dev = float(np.mean(devs))
    achieved = bytes_per_launch / (mean_dev * 1e-3) / 1e9
    log(f"[mla] p50 {pct(walls, 50):.4f} ms  p99 {pct(walls, 99):.4f} ms  "
        f"kernel {mean_dev:.4f} ms  {achieved:.0f} GB/s"
        f"  (timed calls p50 {pct(timed_walls, 50):.4f} ms)")
    log(f"[mla] 1000 calls: p50 {pct(calls_1000, 50):.4f} ms  p99 {pct(calls_1000, 99):.4f} ms")
    return dict(rows=rows, q=q, ids=ids, scores=scores, walls=walls, latent=latent,
                calls_1000=calls_1000,
                timed_p50=pct(timed_walls, 50),
                devs=devs, bytes=bytes_per_launch, achieved=achieved,
                mean_dev=mean_dev, cfg=cfg)


def bench_mla_small(steps: int, warmup: int, cpu_seconds: float, skip_cpu: bool):
    """The 10,000 x 288 fp32 workload, one query, top-3: the GPU route on a
    bank that fits the GPU's caches (11.5 MB; reported as cache-resident,
    not as a fraction of HBM), and the reference's CPU paths on the same
    inputs -- its Python numpy route (core/graft_arena.py:733-801), its
    C++ store route (cpp/grm_runtime.cpp:4299-4361, compiled from the
    reference sources into oracle/_ref when that was built), and the
    oracle's fp64 law on every host thread and on one."""
    import oracle
    from graftrepository_amd import MlaNodeBank, workloads as wl
    from graftrepository_amd.mla_probe import HipProbe

    cfg = wl.MLA_SMALL
    n, d, k = cfg["nodes"], cfg["dim"], cfg["topk"]
    rows = wl.mla_rows(n, d, seed=cfg["seed"])
    q = wl.mla_queries(1, d, seed=cfg["seed"])
    bank = MlaNodeBank(rows)
    probe = HipProbe()
    dq = probe.upload_queries(q)
    for _ in range(warmup):
        bank.route(dq, k, on_device=True, query_count=1)
    walls, devs = [], []
    for _ in range(steps):
        walls.append(bank.route(dq, k, on_device=True, query_count=1, timed=False).wall_ms)
    with route_events():
        for _ in range(min(steps, 300)):
            r = bank.route(dq, k, on_device=True, query_count=1)
            devs.append(r.device_ms)
    host_r = bank.route(q, k, timed=False)
    host_walls = [bank.route(q, k, timed=False).wall_ms for _ in range(min(steps, 300))]
    dq.close()
    bank.close()
    gpu_ids, gpu_sc = r.ids[0].copy(), r.scores[0].copy()
    assert np.array_equal(host_r.ids[0], gpu_ids)
    law_ids, law_sc, _ = oracle.mla_route(rows, q, k)
    law_match = bool(np.array_equal(law_ids[0], gpu_ids)) and bool(
        np.array_equal(law_sc[0].view(np.uint32), gpu_sc.view(np.uint32)))
    np_ids, np_sc, _ = oracle.mla_route_numpy(rows, q, k)
    bank_bytes = n * d * 4 + n * 4
    out = {
        "workload": "mla_route_small", "nodes": n, "dim": d, "bank_dtype": "f32",
        "topk": k, "queries_per_call": 1, "steps": steps,
        "p50_ms": round(pct(walls, 50), 5), "p99_ms": round(pct(walls, 99), 5),
        "host_query_p50_ms": round(pct(host_walls, 50), 5),
        "kernel_ms_mean": round(float(np.mean(devs)), 5),
        "residency": f"cache-resident: the {bank_bytes / 1e6:.1f} MB bank fits the "
                     "GPU's L2/MALL, so no HBM fraction is claimed",
        "effective_gbs": round(bank_bytes / (float(np.mean(devs)) * 1e-3) / 1e9, 1),
        "oracle_fp64_law_match": law_match,
        "python_numpy_law_ids_match": bool(np.array_equal(np_ids[0], gpu_ids.astype(np.int64))),
        "python_numpy_law_max_rel_score_diff": float(np.max(
            np.abs(np_sc[0].astype(np.float64) - gpu_sc) / np.abs(gpu_sc))),
    }
    log(f"[mla 10k] p50 {out['p50_ms']:.4f} ms  p99 {out['p99_ms']:.4f} ms  kernel "
        f"{out['kernel_ms_mean']:.4f} ms (cache-resident)  host-query p50 "
        f"{out['host_query_p50_ms']:.4f} ms  fp64 law match {law_match}  numpy ids match "
        f"{out['python_numpy_law_ids_match']}")
    if skip_cpu:
        return out
    from threadpoolctl import threadpool_info, threadpool_limits

    blas = [i for i in threadpool_info() if i.get("user_api") == "blas"]
    blas_threads = int(blas[0]["num_threads"]) if blas else 1
    t_np = time_cpu(lambda: oracle.mla_route_numpy(rows, q, k), cpu_seconds / 4)
    with threadpool_limits(1):
        t_np1 = time_cpu(lambda: oracle.mla_route_numpy(rows, q, k), cpu_seconds / 4)
    norms = oracle.mla_row_norms(rows)
    nall = cpu_threads_all()
    t_law = time_cpu(lambda: oracle.mla_route_normed(rows, norms, q, k, threads=nall),
                     cpu_seconds / 4)
    t_law1 = time_cpu(lambda: oracle.mla_route_normed(rows, norms, q, k, threads=1),
                      cpu_seconds / 4)
    ref = None
    if oracle.REF_LIB_PATH.exists():
        import oracle.ref as oref
        h = oref.lib().grm_store_create_mla(b"MiniCPM3_TC", 62, 2560, d, 0, d, 0)
        with oref._Store(h) as st:
            for i in range(n):
                st.set_route(st.add_node(), rows[i])
            ref_ids = np.empty(k, dtype=np.uint64)
            import ctypes
            cnt = ctypes.c_uint64()
            q1 = np.ascontiguousarray(q[0])

            def ref_route():
                st._check(oref.lib().grm_store_route(st.h, q1.ctypes.data, d, b"", k,
                                                     ref_ids.ctypes.data, k,
                                                     ctypes.byref(cnt)))
            t_ref = time_cpu(ref_route, cpu_seconds / 4)
            ref = dict(cpu_figure(t_ref, 1), kind="reference",
                       what="grm_store_route of the reference's C++ store (compiled from "
                            "cpp/grm_runtime.cpp); under 32768 entries it runs on one thread "
                            "(cpp/grm_runtime.cpp:4318-4322)",
                       ids_match_gpu=bool(np.array_equal(ref_ids[:cnt.value], gpu_ids)))
    out["cpu_baseline"] = {
        "value": round(pct(t_np, 50), 4), "unit": "ms", "cores": blas_threads,
        "kind": "port",
        "sample": "the full workload: the reference's Python route law restated in numpy "
                  "(fp32 rows @ q, stable sort by -score), p50 over "
                  f"{len(t_np)} single-query calls",
        "python_numpy_law_1_thread": cpu_figure(t_np1, 1),
        "oracle_fp64_law_all_threads": cpu_figure(t_law, nall),
        "oracle_fp64_law_1_thread": cpu_figure(t_law1, 1),
        "reference_store_route": ref,
        "host": host_cpu(),
    }
    log(f"[cpu 10k] numpy law {pct(t_np, 50):.3f} ms ({blas_threads} BLAS threads), "
        f"{pct(t_np1, 50):.3f} ms (1); fp64 law {pct(t_law, 50):.3f} ms ({nall}), "
        f"{pct(t_law1, 50):.3f} ms (1); reference store "
        f"{ref['p50_ms'] if ref else 'not built'} ms")
    return out


def bench_mla_batched(steps: int, warmup: int, cpu_queries: int, traffic: dict | None = None):
    """256 bf16 queries per call on a 1,000,000 x 288 bf16 bank, top-8:
    the matrix-core screen, the certified merge and exact rescore, plus
    any single-query fallbacks, all inside the timed call."""
    import oracle
    from graftrepository_amd import MlaNodeBank, workloads as wl
    from graftrepository_amd.mla_probe import HipProbe

    cfg = wl.MLA_BATCHED
    n, d, nq, k = cfg["nodes"], cfg["dim"], cfg["queries"], cfg["topk"]
    rows = wl.mla_rows(n, d, seed=cfg["seed"], dtype="bf16")
    q = wl.mla_queries(nq, d, seed=cfg["seed"], dtype="bf16")
    bank = MlaNodeBank(rows, dtype="bf16")
    probe = HipProbe()
    dq = probe.upload_queries(q.view(np.float32))  # bf16 bits, uploaded raw
    for _ in range(warmup):
        bank.route(dq, k, on_device=True, query_dtype="bf16", query_count=nq)
    s0 = bank.route_stats()
    walls, devs, screens = [], [], []
    for _ in range(steps):
        r = bank.route(dq, k, on_device=True, query_dtype="bf16", query_count=nq)
        walls.append(r.wall_ms)
        devs.append(r.device_ms)
        screens.append(bank.screen_ms())
    s1 = bank.route_stats()
    dq.close()
    bank.close()
    fallbacks = (s1["fallbacks"] - s0["fallbacks"]) / max(1, steps)
    # parity on a bounded sample of the queries (oracle fp64 law on the host)
    threads = cpu_threads_all()
    sample = min(cpu_queries, nq)
    cpu = None
    if sample > 0:
        rf = oracle.bf16_to_f32(rows).reshape(rows.shape)
        qf = oracle.bf16_to_f32(q[:sample]).reshape(sample, d)
        norms = oracle.mla_row_norms(rf, threads)
        t0 = time.perf_counter()
        ids, sc, _ = oracle.mla_route_normed(rf, norms, qf, k, threads=threads)
        cpu_ms = (time.perf_counter() - t0) * 1e3
        t0 = time.perf_counter()
        oracle.mla_route_normed(rf, norms, qf[:1], k, threads=1)
        one_ms = (time.perf_counter() - t0) * 1e3
        match = bool(np.array_equal(ids, r.ids[:sample])) and bool(
            np.array_equal(sc.view(np.uint32), r.scores[:sample].view(np.uint32)))
        cpu = {"value": round(cpu_ms / sample * nq, 1), "unit": "ms per call",
               "cores": threads, "kind": "port",
               "sample": f"{sample} of the {nq} queries through the oracle's "
                         f"fp64 law on the same bank (row norms precomputed), "
                         f"scaled to {nq}",
               "one_thread": {"value": round(one_ms * nq, 1), "unit": "ms per call",
                              "sample": f"1 of the {nq} queries on 1 thread, scaled to {nq}"},
               "parity_with_gpu": match, "host": host_cpu()}
    flops = 2.0 * nq * n * d
    bytes_screen = n * d * 2 + n * 4
    # the screen kernel bench.py's bank takes: the LDS-ring screen unless
    # GRM_HIP_BATCH_RING=0 selects the previous one (not profiled)
    ring = os.environ.get("GRM_HIP_BATCH_RING", "1") != "0"
    prof = (traffic or {}).get("mla_batch_ring", {}) if ring else {}
    scr = float(np.mean(screens))
    tflops = flops / (scr * 1e-3) / 1e12
    gbs = bytes_screen / (scr * 1e-3) / 1e9
    log(f"[mla-batched] {nq} queries/call  p50 {pct(walls, 50):.4f} ms  "
        f"device {np.mean(devs):.4f} ms  screen {scr:.4f} ms  {tflops:.0f} TFLOP/s  "
        f"{gbs:.0f} GB/s  fallbacks/call {fallbacks:.2f}  "
        f"oracle match {cpu['parity_with_gpu'] if cpu else 'not checked'}")
    return {
        "workload": "mla_batched_route", "nodes": n, "dim": d, "queries_per_call": nq,
        "bank_dtype": "bf16", "query_dtype": "bf16", "topk": k, "steps": steps,
        "p50_ms": round(pct(walls, 50), 5), "p99_ms": round(pct(walls, 99), 5),
        "device_ms_mean": round(float(np.mean(devs)), 5),
        "queries_per_s": round(nq / (pct(walls, 50) * 1e-3), 1),
        "fallbacks_per_call": fallbacks,
        "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": 2500.0,
                     "unit": "TFLOP/s", "frac": round(tflops / 2500.0, 4),
                     "traffic": prof.get("fetch_bytes"),
                     "mfma_util_counters": prof.get("mfma_util"),
                     "kernel": "mla_batch_ring_kernel<18>" if ring else "mla_batch_screen_kernel<18, 8>",
                     "flops_per_launch": flops, "kernel_ms_mean": round(scr, 5)},
        "roofline_hbm": {"achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "bytes_per_launch": bytes_screen},
        "cpu_baseline": cpu,
    }


def cpu_baseline_gqa(keys, offs, kv, hd, q_bits, k, gpu_ids, gpu_scores, seconds):
    """The 512-node ragged route on the host: the oracle's fp64 law
    (gqa_raw_score, cpp/grm_runtime.cpp:2980-3029) on every host thread
    and on one, over the same bf16 keys and query."""
    import oracle
    from graftrepository_amd.node_bank import bf16_bits_to_f32

    qf = bf16_bits_to_f32(q_bits).reshape(q_bits.shape)
    nall = cpu_threads_all()
    res = {}

    def route(th):
        res["r"] = oracle.gqa_route(keys, oracle.BF16, offs, kv, hd, qf, k, threads=th)

    t_all = time_cpu(lambda: route(nall), seconds * 0.6, warmup=1, min_calls=2, max_calls=20)
    ids, sc, _ = res["r"]
    match = bool(np.array_equal(ids[0], gpu_ids)) and bool(
        np.array_equal(sc[0].view(np.uint32), gpu_scores.view(np.uint32)))
    t_one = time_cpu(lambda: route(1), 0.0, warmup=0, min_calls=1)
    log(f"[cpu gqa] fp64 law p50 {pct(t_all, 50):.1f} ms on {nall} threads, "
        f"{pct(t_one, 50):.1f} ms on 1; ids/scores match GPU: {match}")
    return {"value": round(pct(t_all, 50), 3), "unit": "ms", "cores": nall, "kind": "port",
            "sample": f"the full workload: {len(t_all)} routes of the 512-node bank through "
                      "the oracle's fp64 law (OpenMP over nodes), p50",
            "one_thread": cpu_figure(t_one, 1), "parity_with_gpu": match,
            "host": host_cpu()}


def bench_gqa(steps: int, warmup: int, cpu_seconds: float = 0.0):
    from graftrepository_amd import GqaNodeBank, workloads as wl
    from graftrepository_amd.gqa_probe import HipProbe

    cfg = wl.GQA_RAGGED
    kv = cfg["layers"] * cfg["kv_heads"]
    H = cfg["layers"] * cfg["heads"]
    hd = cfg["head_dim"]
    lens = wl.gqa_lengths(cfg["nodes"], cfg["seed"], lo=cfg["lo"], hi=cfg["hi"])
    keys, offs = wl.gqa_bank(lens, kv, hd, cfg["seed"])
    q = wl.gqa_queries(1, H, cfg["tokens"], hd, cfg["seed"])
    bank = GqaNodeBank(keys, offs, kv_heads=kv, head_dim=hd, dtype="bf16")
    probe = HipProbe()
    dq = probe.upload_queries(q.view(np.float32))  # bf16 bits, uploaded raw
    shape = q.shape
    for _ in range(warmup):
        bank.route(dq, cfg["topk"], on_device=True, query_dtype="bf16",
                   query_shape=shape)
    # latency: routes that ask for no device time, as a caller makes them
    # (completion seen through the finalize blocks' flags); device time:
    # the same routes with stream events around the kernels; and the
    # latency of routes that ask for device time (device clock, flags)
    walls, devs = [], []
    for _ in range(steps):
        r = bank.route(dq, cfg["topk"], on_device=True, query_dtype="bf16",
                       query_shape=shape, timed=False)
        walls.append(r.wall_ms)
        ids0, sc0 = r.ids, r.scores
    with route_events():
        for _ in range(min(steps, 300)):
            r = bank.route(dq, cfg["topk"], on_device=True, query_dtype="bf16",
                           query_shape=shape)
            assert np.array_equal(r.ids, ids0) and np.array_equal(r.scores, sc0)
            devs.append(r.device_ms)
    timed_walls = []
    for _ in range(min(steps, 300)):
        r = bank.route(dq, cfg["topk"], on_device=True, query_dtype="bf16",
                       query_shape=shape)
        assert np.array_equal(r.ids, ids0) and np.array_equal(r.scores, sc0)
        timed_walls.append(r.wall_ms)
    dq.close()
    # the same query handed over from host memory (one H2D copy per call,
    # as the drop-in route takes it)
    host_walls = []
    for _ in range(min(steps, 300)):
        r = bank.route(q, cfg["topk"], query_dtype="bf16", timed=False)
        assert np.array_equal(r.ids, ids0) and np.array_equal(r.scores, sc0)
        host_walls.append(r.wall_ms)
    # the same bank with 4 query tokens per head (16 query columns per kv
    # head instead of 4)
    q4 = wl.gqa_queries(1, H, 4, hd, cfg["seed"] + 1)
    dq4 = probe.upload_queries(q4.view(np.float32))
    for _ in range(warmup):
        bank.route(dq4, cfg["topk"], on_device=True, query_dtype="bf16", query_shape=q4.shape)
    walls4 = [bank.route(dq4, cfg["topk"], on_device=True, query_dtype="bf16",
                         query_shape=q4.shape, timed=False).wall_ms
              for _ in range(max(1, steps // 2))]
    with route_events():
        devs4 = [bank.route(dq4, cfg["topk"], on_device=True, query_dtype="bf16",
                            query_shape=q4.shape).device_ms
                 for _ in range(min(steps, 100))]
    dq4.close()
    # a 64-token query (a prompt-length probe key): 256 query columns per
    # kv head, routed in four passes of 64
    q64 = wl.gqa_queries(1, H, 64, hd, cfg["seed"] + 2)
    dq64 = probe.upload_queries(q64.view(np.float32))
    for _ in range(3):
        bank.route(dq64, cfg["topk"], on_device=True, query_dtype="bf16", query_shape=q64.shape)
    walls64 = [bank.route(dq64, cfg["topk"], on_device=True, query_dtype="bf16",
                          query_shape=q64.shape, timed=False).wall_ms
               for _ in range(max(1, steps // 4))]
    with route_events():
        devs64 = [bank.route(dq64, cfg["topk"], on_device=True, query_dtype="bf16",
                             query_shape=q64.shape).device_ms
                  for _ in range(min(steps, 50))]
    dq64.close()
    bank.close()
    sum_l = int(offs[-1])
    bytes_per_call = sum_l * kv * hd * 2
    mean_dev = float(np.mean(devs))
    achieved = bytes_per_call / (mean_dev * 1e-3) / 1e9
    qt4 = {"query_tokens": 4, "p50_ms": round(pct(walls4, 50), 5),
           "device_ms_mean": round(float(np.mean(devs4)), 5),
           "achieved_gbs": round(bytes_per_call / (float(np.mean(devs4)) * 1e-3) / 1e9, 1)}
    d64 = float(np.mean(devs64))
    flops64 = 2.0 * sum_l * kv * (H // kv) * 64 * hd
    t_floor = max(bytes_per_call / (HBM_PEAK_GBS * 1e9), flops64 / 2.5e15)
    qt64 = {"query_tokens": 64, "query_columns_per_kv_head": (H // kv) * 64,
            "p50_ms": round(pct(walls64, 50), 5), "device_ms_mean": round(d64, 5),
            "roofline": {"bound": "hbm", "achieved": round(bytes_per_call / (d64 * 1e-3) / 1e9, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(bytes_per_call / (d64 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                         "bytes_per_call": bytes_per_call, "flops_per_call": flops64,
                         "mfma_tflops": round(flops64 / (d64 * 1e-3) / 1e12, 1),
                         "floor_ms": round(t_floor * 1e3, 5),
                         "frac_of_floor": round(t_floor * 1e3 / d64, 4)}}
    log(f"[gqa qt64] p50 {qt64['p50_ms']:.4f} ms  device {d64:.4f} ms  "
        f"floor {t_floor * 1e3:.4f} ms ({qt64['roofline']['frac_of_floor']:.2f} of it)")
    log(f"[gqa qt4] p50 {qt4['p50_ms']:.4f} ms  device {qt4['device_ms_mean']:.4f} ms"
        f"  {qt4['achieved_gbs']:.0f} GB/s")
    log(f"[gqa] sumL {sum_l}  p50 {pct(walls, 50):.4f} ms  p99 {pct(walls, 99):.4f} ms"
        f"  device {mean_dev:.4f} ms  {achieved:.0f} GB/s"
        f"  (timed calls p50 {pct(timed_walls, 50):.4f} ms, host query p50 {pct(host_walls, 50):.4f} ms)")
    cpu = None
    if cpu_seconds > 0:
        cpu = cpu_baseline_gqa(keys, offs, kv, hd, q, cfg["topk"], ids0[0], sc0[0],
                               cpu_seconds)
    return dict(keys=keys, offs=offs, q=q, ids=r.ids[0].copy(), cpu=cpu,
                scores=r.scores[0].copy(), walls=walls, devs=devs,
                bytes=bytes_per_call, achieved=achieved, mean_dev=mean_dev,
                timed_p50=pct(timed_walls, 50), host_p50=pct(host_walls, 50), qt4=qt4,
                sum_l=sum_l, cfg=cfg, kv=kv, H=H, qt64=qt64)


def bench_gqa_f32_dropin(steps: int, warmup: int, traffic: dict | None = None):
    """The reference's own GQA hand-over at the 512-node ragged shape: a
    dense, zero-padded fp32 bank [nodes, kv, 512, hd] through
    grm_gqa_cuda_arena_create and host fp32 queries through
    grm_gqa_cuda_arena_route (core/grm_cuda_router.py:183-231), timed as
    that caller sees it (query upload included).  The library drops the
    padding and screens the fp16 copy of the keys; the roofline counts the
    copy's bytes over the actual tokens."""
    import oracle
    from graftrepository_amd import workloads as wl
    from graftrepository_amd.grm_hip_router import CudaGQARouteSidecar

    cfg = wl.GQA_RAGGED
    kv = cfg["layers"] * cfg["kv_heads"]
    H = cfg["layers"] * cfg["heads"]
    hd = cfg["head_dim"]
    n = cfg["nodes"]
    lens = wl.gqa_lengths(n, cfg["seed"], lo=cfg["lo"], hi=cfg["hi"])
    keys, offs = wl.gqa_bank(lens, kv, hd, cfg["seed"], dtype="f32")
    T = int(cfg["hi"])
    dense = np.zeros((n, kv, T, hd), dtype=np.float32)
    for i in range(n):
        L = int(lens[i])
        dense[i, :, :L, :] = keys[int(offs[i]) * kv * hd:int(offs[i + 1]) * kv * hd].reshape(kv, L, hd)
    del keys
    q = wl.gqa_queries(1, H, cfg["tokens"], hd, cfg["seed"], dtype="f32")
    sidecar = CudaGQARouteSidecar.build()
    bank = sidecar.create_bank(dense)
    for _ in range(warmup):
        bank.route_topk(q, topk=cfg["topk"])
    # the caller's latency (every call asks for device time: device clock,
    # flags), then the device time with HIP events around the kernels
    walls, devs = [], []
    for _ in range(steps):
        mapped, rec = bank.route_topk(q, topk=cfg["topk"])
        walls.append(rec.route_wall_ms)
    with route_events():
        for _ in range(steps):
            mapped_ev, rec = bank.route_topk(q, topk=cfg["topk"])
            assert np.array_equal(mapped_ev, mapped)
            devs.append(rec.device_route_ms_total)
    setup_ms = bank.setup_wall_ms
    bank.close()
    # parity: the oracle's fp64 law on the dense bank (checker only)
    want, _, _ = oracle.gqa_route(dense.reshape(-1), oracle.F32,
                                  np.arange(n + 1, dtype=np.uint64) * T, kv, hd, q, cfg["topk"])
    parity = bool(np.array_equal(mapped.reshape(-1), want.reshape(-1)))
    del dense
    sum_l = int(np.sum(lens))
    bytes_copy = sum_l * kv * hd * 2          # the screen's fp16 stream
    bytes_f32 = sum_l * kv * hd * 4           # the fp32 bank over actual tokens
    bytes_dense = n * T * kv * hd * 4         # the padded bank handed over
    mean_dev = float(np.mean(devs))
    ach = bytes_copy / (mean_dev * 1e-3) / 1e9
    out = {"workload": "gqa_ragged_route_f32_dropin", "nodes": n, "sum_tokens": sum_l,
           "dense_rows": T, "kv_heads_stacked": kv, "query_heads_stacked": H,
           "head_dim": hd, "bank_dtype": "f32 (dense, zero-padded)", "screen_copy": "f16",
           "query": "host f32, uploaded per call", "topk": cfg["topk"], "steps": steps,
           "p50_ms": round(pct(walls, 50), 5), "p99_ms": round(pct(walls, 99), 5),
           "device_ms_mean": round(mean_dev, 5), "setup_wall_ms": round(setup_ms, 1),
           "oracle_ids_match": parity,
           "bytes": {"fp16_copy_actual_tokens": bytes_copy, "f32_actual_tokens": bytes_f32,
                     "f32_dense_handed_over": bytes_dense},
           "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS,
                        "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
                        "kernel": "gqa_sr_kernel<f16, 4, 1, fp32 rows>",
                        "traffic": (traffic or {}).get("gqa_sr_f32", {}).get("bytes_per_launch"),
                        "bytes_per_call": bytes_copy}}
    log(f"[gqa f32 drop-in] p50 {out['p50_ms']:.4f} ms  device {mean_dev:.4f} ms  "
        f"{ach:.0f} GB/s on the fp16 copy  parity {parity}  setup {setup_ms:.0f} ms")
    return out


def cpu_baseline_gqa_int8(codes, scales, offs, kv, hd, q_bits, k):
    """The 100k-node INT8 route on the host, sampled: the oracle's fp64
    law with the packed format's dequant (fp16(code * scale),
    core/graft_quant.py:136-144) over a leading slice of the bank's nodes
    with all 16 queries, scaled to the bank's token count (the law's work
    is linear in tokens)."""
    import oracle
    from graftrepository_amd.node_bank import bf16_bits_to_f32

    qf = bf16_bits_to_f32(q_bits).reshape(q_bits.shape)
    n = offs.size - 1
    total = int(offs[-1])
    nall = cpu_threads_all()

    def run(m, th):
        t = int(offs[m])
        t0 = time.perf_counter()
        oracle.gqa_route(codes[:t * kv * hd], oracle.I8, offs[:m + 1], kv, hd, qf, k,
                         scales=scales[:t * kv], scale_dtype="f16", group_size=hd,
                         threads=th)
        return (time.perf_counter() - t0) * 1e3, t

    m_all = max(1, n // 100)
    ms_all, tok_all = run(m_all, nall)
    m_one = max(1, n // 2000)
    ms_one, tok_one = run(m_one, 1)
    value = ms_all * total / tok_all
    log(f"[cpu int8] fp64 law {ms_all:.0f} ms for {m_all} nodes on {nall} threads -> "
        f"{value / 1e3:.1f} s per call; 1 thread {ms_one:.0f} ms for {m_one} nodes -> "
        f"{ms_one * total / tok_one / 1e3:.1f} s per call")
    return {"value": round(value, 1), "unit": "ms per call", "cores": nall, "kind": "port",
            "sample": f"the first {m_all} of {n} nodes ({tok_all} of {total} tokens) with all "
                      f"{qf.shape[0]} queries through the oracle's fp64 law, scaled to the "
                      "bank's tokens; parity is covered by the tests, not here",
            "one_thread": {"value": round(ms_one * total / tok_one, 1), "unit": "ms per call",
                           "sample": f"the first {m_one} nodes ({tok_one} tokens), scaled"},
            "host": host_cpu()}


def bench_gqa_int8(steps: int, warmup: int, cpu_seconds: float = 0.0, traffic: dict | None = None):
    """100,000 lognormal-length nodes (median 256, sigma 0.5, cap 4096),
    8 kv heads x 128 stored INT8 with one fp16 scale per row, 32 bf16 query
    heads, 16 queries per call, top-5; 1% of the nodes are evicted and as
    many appended between calls (not timed; reported apart)."""
    from graftrepository_amd import GqaNodeBank, workloads as wl
    from graftrepository_amd.gqa_probe import HipProbe

    cfg = wl.GQA_INT8
    n, kv, hd, H = cfg["nodes"], cfg["kv_heads"] * cfg["layers"], cfg["head_dim"], cfg["heads"]
    lens = wl.gqa_lengths(n, cfg["seed"], kind="lognormal", median=cfg["median"],
                          sigma=cfg["sigma"], cap=cfg["cap"])
    t0 = time.time()
    codes, scales, offs = wl.gqa_int8_bank(lens, kv, hd, seed=cfg["seed"])
    log(f"[int8] generated {codes.size / 1e9:.1f} GB of codes in {time.time() - t0:.1f}s")
    churn = n // 100
    pool = []
    for j in range(3):
        nl = wl.gqa_lengths(churn, 200 + j, kind="lognormal", median=cfg["median"],
                            sigma=cfg["sigma"], cap=cfg["cap"])
        nc, ns, _ = wl.gqa_int8_bank(nl, kv, hd, seed=200 + j)
        pool.append((nl, nc, ns))
    extra = max(int(p[0].sum()) + 7 * churn for p in pool) * (steps + warmup + 1)
    t0 = time.time()
    bank = GqaNodeBank(codes, offs, kv_heads=kv, head_dim=hd, dtype="i8", scales=scales,
                       scale_dtype="f16", group_size=hd, capacity_nodes=n + churn,
                       capacity_tokens=int(offs[-1]) + extra)
    log(f"[int8] bank created in {time.time() - t0:.1f}s")
    q = wl.gqa_queries(cfg["queries"], H, 1, hd, cfg["seed"], dtype="bf16")
    cpu = None
    if cpu_seconds > 0:
        cpu = cpu_baseline_gqa_int8(codes, scales, offs, kv, hd, q, cfg["topk"])
    del codes
    probe = HipProbe()
    dq = probe.upload_queries(q.view(np.float32))
    rng = np.random.default_rng(cfg["seed"])
    live = np.arange(n, dtype=np.uint64)
    next_id = n
    walls, devs, churns, live_tokens = [], [], [], []
    tok_of = {int(i): int(x) for i, x in enumerate(lens)}
    for step in range(warmup + steps):
        r = bank.route(dq, cfg["topk"], on_device=True, query_dtype="bf16", query_shape=q.shape)
        if step >= warmup:
            walls.append(r.wall_ms)
            devs.append(r.device_ms)
            live_tokens.append(sum(tok_of.values()))
        t1 = time.perf_counter()
        pick = rng.choice(live.size, size=churn, replace=False)
        ev = live[pick]
        bank.evict(ev)
        nl, nc, ns = pool[step % 3]
        nid = np.arange(next_id, next_id + churn, dtype=np.uint64)
        next_id += churn
        bank.append(nc, nl, nid, scales=ns)
        bank.sync()
        churns.append((time.perf_counter() - t1) * 1e3)
        for i in ev.tolist():
            del tok_of[i]
        tok_of.update({int(i): int(x) for i, x in zip(nid, nl)})
        live[pick] = nid
    # Steady phase: the same calls back to back on the churned bank.  Each
    # timed call above follows ~20 ms of host-side churn during which the
    # GPU idles, and a call that starts on an idle GPU runs ~20 % longer
    # (clocks ramp back up within the call); in serving, routes interleave
    # with model work instead.  Both phases are reported.
    steady_walls, steady_devs = [], []
    steady_tokens = sum(tok_of.values())
    for _ in range(max(steps, 10)):
        r = bank.route(dq, cfg["topk"], on_device=True, query_dtype="bf16", query_shape=q.shape)
        steady_walls.append(r.wall_ms)
        steady_devs.append(r.device_ms)
    dq.close()
    bank.close()
    mean_dev = float(np.mean(devs))
    bytes_per_call = float(np.mean(live_tokens)) * kv * (hd + 2)
    achieved = bytes_per_call / (mean_dev * 1e-3) / 1e9
    steady_dev = float(np.mean(steady_devs))
    steady_bytes = float(steady_tokens) * kv * (hd + 2)
    steady_gbs = steady_bytes / (steady_dev * 1e-3) / 1e9
    log(f"[int8] p50 {pct(walls, 50):.4f} ms  p99 {pct(walls, 99):.4f} ms  device {mean_dev:.4f} ms"
        f"  {achieved:.0f} GB/s  churn {np.median(churns):.1f} ms")
    log(f"[int8 steady] p50 {pct(steady_walls, 50):.4f} ms  device {steady_dev:.4f} ms  {steady_gbs:.0f} GB/s")
    return {
        "workload": "gqa_int8_route", "nodes": n, "lengths": "lognormal median 256 sigma 0.5 cap 4096",
        "kv_heads": kv, "query_heads": H, "head_dim": hd, "bank_dtype": "i8+f16 row scales",
        "queries_per_call": cfg["queries"], "topk": cfg["topk"], "steps": steps,
        "live_tokens_mean": round(float(np.mean(live_tokens))),
        "p50_ms": round(pct(walls, 50), 5), "p99_ms": round(pct(walls, 99), 5),
        "device_ms_mean": round(mean_dev, 5),
        "churn_ms_p50": round(float(np.median(churns)), 3),
        "cpu_baseline": cpu,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "bytes_per_call": round(bytes_per_call),
                     "screen_kernel": "gqa_smax_kernel<i8, 4, 4, fact, f16>",
                     "screen_traffic": (traffic or {}).get("gqa_int8_smax", {}).get("bytes_per_launch"),
                     "note": "whole route (6 kernels), each call right after a churn step"},
        "steady": {"calls": len(steady_devs), "p50_ms": round(pct(steady_walls, 50), 5),
                   "device_ms_mean": round(steady_dev, 5), "live_tokens": int(steady_tokens),
                   "roofline": {"bound": "hbm", "achieved": round(steady_gbs, 1),
                                "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                "frac": round(steady_gbs / HBM_PEAK_GBS, 4),
                                "bytes_per_call": round(steady_bytes),
                                "note": "whole route, calls back to back on the churned bank"}},
    }


def bench_bridge(epochs: int):
    """Arena-bridge refresh cost: a bank that follows its arena's grafts
    with evictions and appends, against the full rebuild (walk, stack,
    create and upload) the reference runs on every signature change.
    Every epoch retires, adds and replaces about 1% of the nodes."""
    from graftrepository_amd import bank_bridge as bb
    from graftrepository_amd import workloads as wl

    def run(name, bridge, gs, make, walk, churn):
        rng = np.random.default_rng(7)
        nxt = 10_000_000
        bridge.refresh(gs, 0)
        bridge.bank.sync()
        t_ref, t_walk, moved = [], [], []
        for epoch in range(1, epochs + 1):
            live = [g for g in gs if not g.get("retired")]
            pick = rng.choice(len(live), size=2 * churn, replace=False)
            for j in pick[:churn]:
                live[int(j)]["retired"] = True
            for j in pick[churn:]:
                live[int(j)]["cent"] = make()
            for _ in range(churn):
                gs.append({"native_node_id": nxt, "cent": make()})
                nxt += 1
            t0 = time.perf_counter()
            ev = bridge.refresh(gs, epoch)
            bridge.bank.sync()
            t_ref.append(time.perf_counter() - t0)
            moved.append(ev.get("bytes_uploaded", 0))
            t0 = time.perf_counter()
            walk(gs)
            t_walk.append(time.perf_counter() - t0)
        # full rebuild at the final arena state
        t_full = []
        for _ in range(3):
            t0 = time.perf_counter()
            fresh = type(bridge)(dtype=bridge.dtype)
            fresh.refresh(gs, 0)
            fresh.bank.sync()
            t_full.append(time.perf_counter() - t0)
            full_bytes = fresh.last_event["bytes_uploaded"]
            fresh.close()
        nodes = sum(1 for g in gs if not g.get("retired"))
        r = {"nodes": nodes, "churn_per_epoch": f"{churn} retired + {churn} replaced + {churn} added",
             "epochs": epochs,
             "refresh_ms_p50": round(pct(t_ref, 50) * 1e3, 3),
             # the walk alone in the reference's form (signature tuples):
             # what the reference pays per epoch before any stacking
             "reference_walk_ms_p50": round(pct(t_walk, 50) * 1e3, 3),
             "bytes_uploaded_per_refresh": int(np.median(moved)),
             "full_rebuild_ms_p50": round(pct(t_full, 50) * 1e3, 3),
             "full_rebuild_bytes": int(full_bytes),
             "rebuilds_during_epochs": bridge.totals["rebuilt"]}
        log(f"[bridge {name}] refresh p50 {r['refresh_ms_p50']:.2f} ms (reference-form walk "
            f"{r['reference_walk_ms_p50']:.2f}), full rebuild {r['full_rebuild_ms_p50']:.2f} ms, "
            f"{r['bytes_uploaded_per_refresh'] / 1e6:.2f} MB vs {full_bytes / 1e6:.1f} MB uploaded")
        bridge.close()
        return r

    rng = np.random.default_rng(3)
    n, dim = 100_000, 288
    rows = wl.mla_rows(n, dim, seed=11)
    gs = [{"native_node_id": i, "cent": rows[i]} for i in range(n)]
    mk = lambda: wl.normalise_rows(rng.standard_normal((1, dim), dtype=np.float32))[0]
    mla = run("mla", bb.MlaRouteBankBridge(), gs, mk, bb.mla_bank_walk, n // 100 // 3)

    cfg = wl.GQA_RAGGED
    kv, hd = cfg["kv_heads"], cfg["head_dim"]
    lens = wl.gqa_lengths(cfg["nodes"], cfg["seed"], lo=cfg["lo"], hi=cfg["hi"])
    gs = [{"native_node_id": i,
           "cent": rng.standard_normal((kv, int(L), hd), dtype=np.float32)}
          for i, L in enumerate(lens)]
    mkg = lambda: rng.standard_normal((kv, int(rng.integers(cfg["lo"], cfg["hi"] + 1)), hd),
                                      dtype=np.float32)
    gqa = run("gqa", bb.GqaRouteBankBridge(), gs, mkg, bb.gqa_bank_walk, 2)
    return {"mla": dict(mla, dim=dim, bank_dtype="f32"),
            "gqa": dict(gqa, kv_heads=kv, head_dim=hd, lengths="U[16,512]",
                        bank_dtype="f32")}


def bench_store(steps: int):
    """The store route on the device (lexical bonus + route filters,
    grm_store_route_filtered's law) on a 1M x 288 fp32 store, against the
    same store's route without lexical keys or filters."""
    from graftrepository_amd import workloads as wl
    from graftrepository_amd.store_route import DeviceRouteStore, _KNOWN

    n, d = 1_000_000, 288
    rng = np.random.default_rng(17)
    rows = wl.mla_rows(n, d, seed=23)
    vocab = [f"w{i}" for i in range(1000)]
    lex = [[] for _ in range(n)]
    for i in rng.choice(n, size=n // 100, replace=False):
        lex[int(i)] = list(rng.choice(vocab, size=3, replace=False))
    kinds = np.asarray(_KNOWN["kind"])[rng.integers(0, 8, size=n)]
    meta = [(str(k), "", "", "") for k in kinds]
    t0 = time.perf_counter()
    st = DeviceRouteStore(d, capacity=n)
    st.set_routes(np.arange(n, dtype=np.uint64), rows, lex, meta)
    build_s = time.perf_counter() - t0
    q = wl.mla_queries(1, d, seed=29)[0]
    qlex = ["w1", "w2", "w3"]
    walls, plain = [], []
    for i in range(steps + 5):
        t0 = time.perf_counter()
        st.route_filtered(q, qlex, kinds=["turn", "doc"], topk=8)
        t1 = time.perf_counter()
        st.route_scored(q, (), 8)
        t2 = time.perf_counter()
        if i >= 5:
            walls.append((t1 - t0) * 1e3)
            plain.append((t2 - t1) * 1e3)
    st.close()
    r = {"nodes": n, "dim": d, "lexical_nodes": n // 100, "query_lexical": 3,
         "filter": "kind in {turn, doc}", "topk": 8,
         "store_route_ms_p50": round(pct(walls, 50), 4),
         "plain_route_ms_p50": round(pct(plain, 50), 4),
         "build_s": round(build_s, 2)}
    log(f"[store] filtered + lexical route p50 {r['store_route_ms_p50']:.3f} ms "
        f"(plain route {r['plain_route_ms_p50']:.3f} ms), bulk build {build_s:.1f}s")
    return r


def bench_payload(reps: int):
    """Packed graft payloads: the device unpack kernel against its HBM
    roofline, and mounting one packed node payload (device unpack) against
    the reference's route (host dequant, then the fp16 upload)."""
    import ctypes

    import oracle
    from graftrepository_amd import _lib, payload as pl

    lib = _lib.load()
    gs = 32
    # kernel: 1 Gi values, codes + scales + fp16 out = 3.125 B per value
    n = 1 << 30
    block = np.random.default_rng(1).integers(-128, 128, size=64 << 20, dtype=np.int8)
    d_c, d_s, d_o = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
    for ptr, nbytes in ((d_c, n), (d_s, n // gs * 4), (d_o, 2 * n)):
        _lib.check(lib.grm_hip_device_alloc(nbytes, ctypes.byref(ptr)), "alloc")
    try:
        for off in range(0, n, block.size):
            _lib.check(lib.grm_hip_copy_to_device(d_c.value + off, block.ctypes.data,
                                                  block.size), "h2d")
        sc = (np.random.default_rng(2).random(n // gs) * 0.05).astype(np.float32)
        _lib.check(lib.grm_hip_copy_to_device(d_s.value, sc.ctypes.data, sc.nbytes), "h2d")
        ms = ctypes.c_float()
        times = []
        for i in range(reps + 2):
            _lib.check(lib.grm_hip_payload_dequant(d_c, d_s, n, gs, d_o, ctypes.byref(ms)),
                       "dequant")
            if i >= 2:
                times.append(ms.value)
    finally:
        for ptr in (d_c, d_s, d_o):
            lib.grm_hip_device_free(ptr)
    bytes_per_launch = n * (1 + 4 / gs + 2)
    kms = float(np.mean(times))
    achieved = bytes_per_launch / (kms * 1e-3) / 1e9
    log(f"[payload] unpack kernel {kms:.3f} ms for {n} values: {achieved:.0f} GB/s")

    # mount of one packed node payload (L, H, S, D) = (28, 4, 512, 128), k and v
    rng = np.random.default_rng(3)
    shape = (28, 4, 512, 128)
    arrays = {nm: (rng.standard_normal(shape) * 2).astype(np.float16) for nm in ("k", "v")}
    z = {"format_version": np.asarray(1, np.int64), "storage_bits": np.asarray(8, np.int64),
         "group_size": np.asarray(gs, np.int64)}
    for nm, a in arrays.items():
        c, s_ = oracle.quantize_symmetric(a, 8, gs)
        z[f"{nm}_codes"], z[f"{nm}_scales"] = c, s_
        z[f"{nm}_shape"] = np.asarray(a.shape, np.int64)
    dev, host = [], []
    for i in range(reps + 2):
        t0 = time.perf_counter()
        out = pl.unpack_node_device(z)
        t1 = time.perf_counter()
        for a in out.values():
            a.close()
        # the reference's route: numpy dequant (core/graft_quant.py:136-144),
        # then the fp16 arrays uploaded
        t2 = time.perf_counter()
        ups = []
        for nm in ("k", "v"):
            h = (z[f"{nm}_codes"].astype(np.float32) * z[f"{nm}_scales"]).reshape(shape)
            h = h.astype(np.float16)
            d = pl.DeviceArray(shape)
            _lib.check(lib.grm_hip_copy_to_device(d.ptr, h.ctypes.data, h.nbytes), "h2d")
            ups.append(d)
        t3 = time.perf_counter()
        for d in ups:
            d.close()
        if i >= 2:
            dev.append(t1 - t0)
            host.append(t3 - t2)
    vals = 2 * int(np.prod(shape))
    r = {"unpack_kernel": {"values": n, "group_size": gs, "device_ms_mean": round(kms, 4),
                           "bytes_per_launch": int(bytes_per_launch),
                           "roofline": {"bound": "hbm", "achieved": round(achieved, 1),
                                        "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                        "frac": round(achieved / HBM_PEAK_GBS, 4)}},
         "node_mount": {"shape_each": list(shape), "tensors": ["k", "v"], "storage_bits": 8,
                        "device_unpack_ms_p50": round(pct(dev, 50) * 1e3, 3),
                        "host_dequant_then_fp16_upload_ms_p50": round(pct(host, 50) * 1e3, 3),
                        "bytes_crossing_pcie_packed": int(vals * (1 + 4 / gs)),
                        "bytes_crossing_pcie_fp16": 2 * vals}}
    log(f"[payload] node mount {r['node_mount']['device_unpack_ms_p50']:.2f} ms packed "
        f"vs {r['node_mount']['host_dequant_then_fp16_upload_ms_p50']:.2f} ms host dequant + fp16")
    return r


def cpu_baseline_mla(m, seconds: float):
    """The 1M x 288 route on the host: the oracle's fp64 law with the row
    norms held as the reference's arena holds them (the route's per-call
    work, cpp/grm_runtime.cpp:4299-4361) on every host thread and on one,
    and the reference's Python numpy law (core/graft_arena.py:778-801) at
    the BLAS library's thread count and on one thread."""
    import oracle
    from threadpoolctl import threadpool_info, threadpool_limits

    rows, q, k = m["rows"], m["q"], m["cfg"]["topk"]
    nall = cpu_threads_all()
    norms = oracle.mla_row_norms(rows, nall)
    res = {}

    def law(th):
        res["law"] = oracle.mla_route_normed(rows, norms, q, k, threads=th)

    t_all = time_cpu(lambda: law(nall), seconds * 0.5, warmup=2)
    ids, sc, _ = res["law"]
    match = bool(np.array_equal(ids[0], m["ids"])) and bool(
        np.array_equal(sc[0].view(np.uint32), m["scores"].view(np.uint32)))
    t_one = time_cpu(lambda: law(1), seconds * 0.2, warmup=1, min_calls=2)
    blas = [i for i in threadpool_info() if i.get("user_api") == "blas"]
    blas_threads = int(blas[0]["num_threads"]) if blas else 1
    t_np = time_cpu(lambda: oracle.mla_route_numpy(rows, q, k), seconds * 0.15, warmup=2)
    with threadpool_limits(1):
        t_np1 = time_cpu(lambda: oracle.mla_route_numpy(rows, q, k), seconds * 0.15,
                         warmup=1, min_calls=2)
    np_ids, _, _ = oracle.mla_route_numpy(rows, q, k)
    log(f"[cpu 1M] fp64 law p50 {pct(t_all, 50):.1f} ms on {nall} threads, "
        f"{pct(t_one, 50):.1f} ms on 1; numpy law {pct(t_np, 50):.1f} ms "
        f"({blas_threads} BLAS threads), {pct(t_np1, 50):.1f} ms on 1; "
        f"ids/scores match GPU: {match}")
    return dict(value=round(pct(t_all, 50), 3), unit="ms", cores=nall, kind="port",
                sample=f"the full workload: {len(t_all)} single-query routes of the "
                       "1,000,000 x 288 bank through the oracle's fp64 law (OpenMP; row "
                       "norms precomputed as the reference's arena keeps them), p50",
                parity_with_gpu=match,
                fp64_law_1_thread=cpu_figure(t_one, 1),
                python_numpy_law=dict(cpu_figure(t_np, blas_threads),
                                      ids_match_gpu=bool(np.array_equal(
                                          np_ids[0], m["ids"].astype(np.int64)))),
                python_numpy_law_1_thread=cpu_figure(t_np1, 1),
                host=host_cpu())


def reference_router_mla(rows, q, k, gpu_ids, seconds: float):
    """The reference's own CPU router on the full 1M x 288 bank:
    grm_store_route of its C++ store (cpp/grm_runtime.cpp:6767-6825 ->
    route_mla_arena, :4299-4361), compiled from its sources into
    oracle/_ref.  At 1M entries it scores with OpenMP over entries
    (:4318-4322) on the process's OpenMP threads.  The store's first route
    builds its snapshot and arena; that is reported apart and not timed."""
    import ctypes

    import oracle
    import oracle.ref as oref

    if not oracle.REF_LIB_PATH.exists():
        return None
    n, d = rows.shape
    L = oref.lib()
    t0 = time.perf_counter()
    st = oref._Store(L.grm_store_create_mla(b"MiniCPM3_TC", 62, 2560, d, 0, d, 0))
    try:
        nid = ctypes.c_uint64()
        for i in range(n):
            st._check(L.grm_store_add_node(st.h, b"n", 1, None, 0, ctypes.byref(nid)))
            st._check(L.grm_store_set_route(st.h, nid.value, rows[i].ctypes.data, d, b""))
            if (i + 1) % 250_000 == 0:
                log(f"[ref mla] {i + 1} entries stored ({time.perf_counter() - t0:.0f}s)")
        load_s = time.perf_counter() - t0
        out = np.empty(k, dtype=np.uint64)
        cnt = ctypes.c_uint64()
        q1 = np.ascontiguousarray(q[0], dtype=np.float32)

        def route():
            st._check(L.grm_store_route(st.h, q1.ctypes.data, d, b"", k, out.ctypes.data, k,
                                        ctypes.byref(cnt)))

        t0 = time.perf_counter()
        route()
        first_ms = (time.perf_counter() - t0) * 1e3
        times = time_cpu(route, seconds, warmup=1, min_calls=3, max_calls=20)
        match = bool(np.array_equal(out[:cnt.value], gpu_ids))
    finally:
        st.close()
    r = dict(cpu_figure(times, cpu_threads_all()), kind="reference",
             what="grm_store_route of the reference's C++ store, compiled from "
                  "cpp/grm_runtime.cpp into oracle/_ref; OpenMP over the 1,000,000 entries "
                  "(cpp/grm_runtime.cpp:4318-4322)",
             sample="the full workload", ids_match_gpu=match,
             store_load_s=round(load_s, 1), first_route_ms=round(first_ms, 1))
    log(f"[ref mla] grm_store_route p50 {r['p50_ms']:.1f} ms on {r['threads']} threads "
        f"(load {load_s:.0f}s, first route {first_ms:.0f} ms), ids match GPU: {match}")
    return r


def reference_router_gqa(keys_bits, offs, kv, hd, q_bits, k, seconds: float,
                         sample_nodes: int = 128):
    """The reference's own CPU router on the ragged bank, sampled:
    grm_store_route_gqa (cpp/grm_runtime.cpp:6898-6961 -> route_gqa_raw,
    :4498-4881) over one fp32 key [kv, L_i, hd] per node (the bf16 keys,
    widened), which takes its default fp32 arena path
    (gqa_arena_key_score, :3588-3671).  Its route time is linear in the
    bank's tokens, but its arena build (the first route after a change)
    reserves each key's rows exactly (:3350), so it copies the arena once
    per key and grows with the square of the node count: over two minutes
    at 512 nodes.  The store therefore holds the first `sample_nodes`
    nodes, the route is timed on them and scaled to the whole bank's
    tokens, and its ids are checked against the oracle's fp64 law on the
    same sample."""
    import ctypes

    import oracle
    import oracle.ref as oref
    from graftrepository_amd.node_bank import bf16_bits_to_f32

    if not oracle.REF_LIB_PATH.exists():
        return None
    L = oref.lib()
    H, Qt = q_bits.shape[1], q_bits.shape[2]
    qf = np.ascontiguousarray(bf16_bits_to_f32(q_bits).reshape(H, Qt, hd))
    m = min(sample_nodes, offs.size - 1)
    st = oref._Store(L.grm_store_create_gqa(b"Qwen3_TC", 36, 2560, 2 * kv * hd, 0, kv, hd))
    try:
        for i in range(m):
            a, b = int(offs[i]), int(offs[i + 1])
            blk = bf16_bits_to_f32(keys_bits[a * kv * hd:b * kv * hd]).reshape(kv, b - a, hd)
            st.set_route_list(st.add_node(), [blk])
        out = np.empty(k, dtype=np.uint64)
        cnt = ctypes.c_uint64()

        def route():
            st._check(L.grm_store_route_gqa(st.h, qf.ctypes.data, H, Qt, hd, b"", b"", b"", b"",
                                            b"", k, out.ctypes.data, k, ctypes.byref(cnt)))

        t0 = time.perf_counter()
        route()
        first_ms = (time.perf_counter() - t0) * 1e3
        times = time_cpu(route, seconds, warmup=1, min_calls=3, max_calls=50)
        got = out[:cnt.value].copy()
    finally:
        st.close()
    tok_s, tok = int(offs[m]), int(offs[-1])
    law_ids, _, _ = oracle.gqa_route(keys_bits[:tok_s * kv * hd], oracle.BF16, offs[:m + 1],
                                     kv, hd, qf[None], k)
    match = bool(np.array_equal(got, law_ids[0]))
    scale = tok / tok_s
    r = {"value": round(pct(times, 50) * scale, 3), "unit": "ms", "threads": cpu_threads_all(),
         "kind": "reference",
         "what": "grm_store_route_gqa of the reference's C++ store, compiled from "
                 "cpp/grm_runtime.cpp into oracle/_ref; its default fp32 arena path "
                 "(cpp/grm_runtime.cpp:3588-3671, 4498-4881)",
         "sample": f"the first {m} of {offs.size - 1} nodes ({tok_s} of {tok} tokens), "
                   f"p50 over {len(times)} routes scaled by the token ratio {scale:.3f}",
         "sample_p50_ms": round(pct(times, 50), 3), "sample_p95_ms": round(pct(times, 95), 3),
         "ids_match_oracle_on_sample": match, "first_route_ms": round(first_ms, 1)}
    log(f"[ref gqa] grm_store_route_gqa {r['sample_p50_ms']:.2f} ms on {m} nodes -> "
        f"{r['value']:.1f} ms for the bank on {r['threads']} threads (first route "
        f"{first_ms:.0f} ms), ids match the fp64 law on the sample: {match}")
    return r


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--gqa-steps", type=int, default=300)
    ap.add_argument("--batched-steps", type=int, default=100)
    ap.add_argument("--int8-steps", type=int, default=20)
    ap.add_argument("--bridge-epochs", type=int, default=10)
    ap.add_argument("--payload-reps", type=int, default=10)
    ap.add_argument("--store-steps", type=int, default=100)
    ap.add_argument("--small-steps", type=int, default=1000)
    ap.add_argument("--f32-steps", type=int, default=200)
    ap.add_argument("--only", choices=["all", "mla", "small", "gqa", "f32", "batched", "int8",
                                       "bridge", "payload", "store"], default="all")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run the 1 GiB device copy used to scale counters")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures the route on one GPU only; --gpus {args.gpus} "
              f"(WORLD_SIZE {world}) is not supported: the route runs on one "
              "GPU's bank and multi-GPU sharding is not part of this build.",
              file=sys.stderr)
        return 2

    if args.copy_calibration:
        print(json.dumps(copy_calibration()), flush=True)
        return 0

    traffic = load_traffic()
    out = {}
    m = g = None
    if args.only in ("all", "mla"):
        m = bench_mla(args.steps, args.warmup)
    cpu_s = 0.0 if args.skip_cpu else args.cpu_seconds
    small = None
    if args.only in ("all", "small"):
        small = bench_mla_small(args.small_steps, min(args.warmup, 20), cpu_s, args.skip_cpu)
    if args.only in ("all", "gqa"):
        g = bench_gqa(args.gqa_steps, min(args.warmup, 20), cpu_s)
    f32 = None
    if args.only in ("all", "f32"):
        f32 = bench_gqa_f32_dropin(args.f32_steps, min(args.warmup, 10), traffic)
    i8 = None
    if args.only in ("all", "int8"):
        i8 = bench_gqa_int8(args.int8_steps, 2, cpu_s, traffic)
    b = None
    if args.only in ("all", "batched"):
        b = bench_mla_batched(args.batched_steps, min(args.warmup, 5),
                              0 if args.skip_cpu else 4, traffic)
    br = None
    if args.only in ("all", "bridge"):
        br = bench_bridge(args.bridge_epochs)
    pay = None
    if args.only in ("all", "payload"):
        pay = bench_payload(args.payload_reps)
    sto = None
    if args.only in ("all", "store"):
        sto = bench_store(args.store_steps)
    cpu = None
    if m is not None and not args.skip_cpu:
        cpu = cpu_baseline_mla(m, args.cpu_seconds)
    if not args.skip_cpu:
        # the reference's own CPU router, after every GPU leg
        if g is not None and g["cpu"] is not None:
            g["cpu"]["reference_router"] = reference_router_gqa(
                g["keys"], g["offs"], g["kv"], g["cfg"]["head_dim"], g["q"],
                g["cfg"]["topk"], args.cpu_seconds * 0.3)
        if cpu is not None:
            cpu["reference_router"] = reference_router_mla(
                m["rows"], m["q"], m["cfg"]["topk"], m["ids"], args.cpu_seconds * 0.5)

    if m is not None:
        cfg = m["cfg"]
        out = {
            "metric": "p50 route latency (ms) @1M MLA nodes + achieved HBM GB/s; ragged GQA p50",
            "value": round(pct(m["walls"], 50), 5),
            "unit": "ms",
            "n_gpus": 1,
            "steps": args.steps,
            "warmup": args.warmup,
            "ms_per_step": round(float(np.mean(m["walls"])), 5),
            "higher_is_better": False,
            "scaling": "weak",
            "vs_baseline": None,
            "dtype": "f64",
            "data": "synthetic (unit-norm Gaussian centroids, seeded)",
            "config": {"workload": "mla_route", "nodes": cfg["nodes"],
                       "dim": cfg["dim"], "bank_dtype": "f32", "topk": cfg["topk"],
                       "queries_per_call": 1, "query_resident": "hbm"},
            "p99_ms": round(pct(m["walls"], 99), 5),
            "calls_1000": {"p50_ms": round(pct(m["calls_1000"], 50), 5),
                           "p99_ms": round(pct(m["calls_1000"], 99), 5),
                           "calls": len(m["calls_1000"])},
            "kernel_ms_mean": round(m["mean_dev"], 5),
            "timed_calls_p50_ms": round(m["timed_p50"], 5),
            "latent_entry": m["latent"],
            "roofline": {"bound": "hbm", "achieved": round(m["achieved"], 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(m["achieved"] / HBM_PEAK_GBS, 4),
                         "traffic": traffic.get("mla_route", {}).get("bytes_per_launch"),
                         "kernel": "mla_route_pipe_kernel<f32, 16, 9>",
                         "bytes_per_launch": m["bytes"]},
        }
    if g is not None:
        gq = {
            "workload": "gqa_ragged_route", "nodes": g["cfg"]["nodes"],
            "sum_tokens": g["sum_l"], "kv_heads_stacked": g["kv"],
            "query_heads_stacked": g["H"], "head_dim": g["cfg"]["head_dim"],
            "bank_dtype": "bf16", "topk": g["cfg"]["topk"],
            "steps": args.gqa_steps,
            "p50_ms": round(pct(g["walls"], 50), 5),
            "p99_ms": round(pct(g["walls"], 99), 5),
            "device_ms_mean": round(g["mean_dev"], 5),
            "timed_calls_p50_ms": round(g["timed_p50"], 5),
            "host_query_p50_ms": round(g["host_p50"], 5),
            "query_tokens_4": dict(g["qt4"], roofline={
                "bound": "hbm", "achieved": g["qt4"]["achieved_gbs"], "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(g["qt4"]["achieved_gbs"] / HBM_PEAK_GBS, 4),
                "traffic": traffic.get("gqa_sr_qt4", {}).get("bytes_per_launch"),
                "kernel": "gqa_sr_kernel<bf16, 4, 1>", "bytes_per_call": g["bytes"]}),
            "query_tokens_64": g["qt64"],
            "cpu_baseline": g["cpu"],
            "roofline": {"bound": "hbm", "achieved": round(g["achieved"], 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(g["achieved"] / HBM_PEAK_GBS, 4),
                         "traffic": traffic.get("gqa_sr", {}).get("bytes_per_launch"),
                         "kernel": "gqa_sr_kernel<bf16, 4, 1>",
                         "bytes_per_call": g["bytes"]},
        }
        if out:
            out["gqa"] = gq
        else:
            out = {"metric": "ragged GQA p50 route latency (ms)",
                   "value": gq["p50_ms"], "unit": "ms", "n_gpus": 1,
                   "steps": args.gqa_steps, "warmup": args.warmup,
                   "ms_per_step": round(float(np.mean(g["walls"])), 5),
                   "higher_is_better": False, "scaling": "weak",
                   "vs_baseline": None, "dtype": "f64",
                   "data": "synthetic", "config": gq}
    if small is not None:
        if out:
            out["mla_small"] = small
        else:
            out = {"metric": "p50 route latency (ms), 10,000 x 288 MLA nodes (cache-resident)",
                   "value": small["p50_ms"], "unit": "ms", "n_gpus": 1,
                   "steps": args.small_steps, "warmup": args.warmup,
                   "ms_per_step": small["p50_ms"], "higher_is_better": False,
                   "scaling": "weak", "vs_baseline": None, "dtype": "f64",
                   "data": "synthetic", "config": small}
            if small.get("cpu_baseline"):
                out["cpu_baseline"] = small["cpu_baseline"]
    if b is not None:
        if out:
            out["mla_batched"] = b
        else:
            out = {"metric": "p50 batched MLA route latency (ms per 256-query call)",
                   "value": b["p50_ms"], "unit": "ms", "n_gpus": 1,
                   "steps": args.batched_steps, "warmup": args.warmup,
                   "ms_per_step": b["p50_ms"], "higher_is_better": False,
                   "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
                   "data": "synthetic", "config": b}
    if f32 is not None:
        if out:
            out["gqa_f32_dropin"] = f32
        else:
            out = {"metric": "p50 ragged GQA route latency (ms), dense fp32 bank, host query",
                   "value": f32["p50_ms"], "unit": "ms", "n_gpus": 1,
                   "steps": args.f32_steps, "warmup": args.warmup,
                   "ms_per_step": f32["p50_ms"], "higher_is_better": False,
                   "scaling": "weak", "vs_baseline": None, "dtype": "f64",
                   "data": "synthetic", "config": f32}
    if i8 is not None:
        if out:
            out["gqa_int8"] = i8
        else:
            out = {"metric": "p50 INT8 ragged GQA route latency (ms per 16-query call)",
                   "value": i8["p50_ms"], "unit": "ms", "n_gpus": 1,
                   "steps": args.int8_steps, "warmup": 2, "ms_per_step": i8["p50_ms"],
                   "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
                   "dtype": "f64", "data": "synthetic", "config": i8}
    if br is not None:
        if out:
            out["bank_bridge"] = br
        else:
            out = {"metric": "arena-bridge refresh p50 (ms) at 1% churn, 100k MLA nodes",
                   "value": br["mla"]["refresh_ms_p50"], "unit": "ms", "n_gpus": 1,
                   "steps": args.bridge_epochs, "warmup": 0,
                   "ms_per_step": br["mla"]["refresh_ms_p50"], "higher_is_better": False,
                   "scaling": "weak", "vs_baseline": None, "dtype": "f32",
                   "data": "synthetic", "config": {"workload": "bank_bridge", **br}}
    if pay is not None:
        if out:
            out["payload"] = pay
        else:
            out = {"metric": "packed payload unpack kernel GB/s (1 Gi values, group 32)",
                   "value": pay["unpack_kernel"]["roofline"]["achieved"], "unit": "GB/s",
                   "n_gpus": 1, "steps": args.payload_reps, "warmup": 2,
                   "ms_per_step": pay["unpack_kernel"]["device_ms_mean"],
                   "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
                   "dtype": "int8->f16", "data": "synthetic",
                   "config": {"workload": "payload_unpack", **pay}}
    if sto is not None:
        if out:
            out["store_route"] = sto
        else:
            out = {"metric": "p50 store route latency (ms), lexical + filters, 1M MLA nodes",
                   "value": sto["store_route_ms_p50"], "unit": "ms", "n_gpus": 1,
                   "steps": args.store_steps, "warmup": 5,
                   "ms_per_step": sto["store_route_ms_p50"], "higher_is_better": False,
                   "scaling": "weak", "vs_baseline": None, "dtype": "f64",
                   "data": "synthetic", "config": {"workload": "store_route", **sto}}
    if cpu is not None:
        out["cpu_baseline"] = cpu
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
