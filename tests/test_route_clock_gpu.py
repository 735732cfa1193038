"""Timed routes on the flag path: device time from the device's constant clock.

A caller that asks for device time (every call through the reference ABI,
grm_{mla,gqa}_cuda_arena_route, core/grm_cuda_router.py:183-231) gets its
results through the finalize blocks' completion flags, as an untimed route
does; the device time is the constant-rate clock's ticks from the first
timed kernel's start to the last flagged block's end instead of stream
events around the kernels (GRM_HIP_ROUTE_TIMING=events restores the
events).  Results must be the oracle's in both modes, and the two device
times must describe the same kernels.
"""

import numpy as np
import pytest

import oracle
from graftrepository_amd import GqaNodeBank, MlaNodeBank
from graftrepository_amd.grm_hip_router import CudaGQARouteSidecar, CudaMLARouteSidecar

pytestmark = pytest.mark.gpu
NO_ID = np.iinfo(np.uint64).max


def assert_same(res_ids, res_scores, want_ids, want_scores):
    np.testing.assert_array_equal(res_ids, want_ids)
    filled = want_ids != NO_ID
    np.testing.assert_array_equal(res_scores[filled].view(np.uint32),
                                  want_scores[filled].view(np.uint32))


def set_timing(monkeypatch, mode):
    if mode == "events":
        monkeypatch.setenv("GRM_HIP_ROUTE_TIMING", "events")
    else:
        monkeypatch.delenv("GRM_HIP_ROUTE_TIMING", raising=False)


def ragged(rng, n, kv, hd, lo, hi):
    lens = rng.integers(lo, hi + 1, size=n).astype(np.uint64)
    offs = np.zeros(n + 1, np.uint64)
    offs[1:] = np.cumsum(lens)
    keys = rng.standard_normal(int(offs[-1]) * kv * hd).astype(np.float32)
    return keys, offs


def agree(clock_ms, event_ms):
    # same kernels, two clocks: the events also hold the launch gaps around
    # them, so the clock's figure may be a little shorter
    return 0.4 * event_ms - 0.02 <= clock_ms <= 1.5 * event_ms + 0.02


@pytest.mark.parametrize("q_count,warmup,Qt", [(1, 0, 1), (4, 1, 1), (3, 2, 4)])
def test_gqa_timed_route_on_the_device_clock(hip_lib, monkeypatch, q_count, warmup, Qt):
    monkeypatch.setenv("GRM_HIP_GQA_SCREEN", "1")
    monkeypatch.setenv("GRM_HIP_GQA_BOUND", "0")
    rng = np.random.default_rng(700 + 10 * q_count + Qt)
    kv, hd, H = 8, 128, 32
    keys, offs = ragged(rng, 300, kv, hd, 16, 400)
    qs = rng.standard_normal((q_count, H, Qt, hd)).astype(np.float32)
    want_ids, want_sc, _ = oracle.gqa_route(oracle.bf16_bits(keys), oracle.BF16, offs, kv, hd, qs, 5)
    dev = {}
    for mode in ("clock", "events"):
        set_timing(monkeypatch, mode)
        with GqaNodeBank(keys, offs, kv_heads=kv, head_dim=hd, dtype="bf16") as bank:
            times = []
            for _ in range(5):
                res = bank.route(qs, 5, warmup=warmup)
                assert_same(res.ids, res.scores, want_ids, want_sc)
                times.append(res.device_ms)
            untimed = bank.route(qs, 5, warmup=warmup, timed=False)
            assert_same(untimed.ids, untimed.scores, want_ids, want_sc)
            stats = bank.route_stats()
        assert stats["screen_refine"] > 0 and stats["exact"] == 0
        assert all(t > 0.0 and np.isfinite(t) for t in times)
        dev[mode] = float(np.median(times))
    assert agree(dev["clock"], dev["events"]), dev


def test_gqa_dropin_route_on_the_device_clock(hip_lib, monkeypatch):
    # the reference's hand-over: dense zero-padded fp32 bank, host queries,
    # device time always asked for
    set_timing(monkeypatch, "clock")
    rng = np.random.default_rng(71)
    n, kv, T, hd, H = 64, 4, 96, 128, 16
    dense = np.zeros((n, kv, T, hd), np.float32)
    lens = rng.integers(1, T + 1, size=n)
    for i in range(n):
        dense[i, :, :lens[i]] = rng.standard_normal((kv, lens[i], hd))
    q = rng.standard_normal((2, H, 1, hd)).astype(np.float32)
    bank = CudaGQARouteSidecar.build().create_bank(dense)
    try:
        mapped, rec = bank.route_topk(q, topk=4, warmup=1, route_repeats=3)
    finally:
        bank.close()
    want, _, _ = oracle.gqa_route(dense.reshape(-1), oracle.F32,
                                  np.arange(n + 1, dtype=np.uint64) * T, kv, hd, q, 4)
    np.testing.assert_array_equal(mapped, want)
    assert all(t > 0.0 for t in rec.device_route_ms_runs)
    assert rec.measured_queries == 1


@pytest.mark.parametrize("q_count,warmup", [(1, 0), (3, 1)])
def test_mla_timed_route_on_the_device_clock(hip_lib, monkeypatch, q_count, warmup):
    rng = np.random.default_rng(900 + q_count)
    n, dim = 200_000, 288
    rows = rng.standard_normal((n, dim)).astype(np.float32)
    qs = rng.standard_normal((q_count, dim)).astype(np.float32)
    want_ids, want_sc, _ = oracle.mla_route(rows, qs, 8)
    dev = {}
    for mode in ("clock", "events"):
        set_timing(monkeypatch, mode)
        with MlaNodeBank(rows) as bank:
            times = []
            for _ in range(5):
                res = bank.route(qs, 8, warmup=warmup)
                assert_same(res.ids, res.scores, want_ids, want_sc)
                times.append(res.device_ms)
        assert all(t > 0.0 and np.isfinite(t) for t in times)
        dev[mode] = float(np.median(times))
    assert agree(dev["clock"], dev["events"]), dev


def test_mla_dropin_route_on_the_device_clock(hip_lib, monkeypatch):
    set_timing(monkeypatch, "clock")
    rng = np.random.default_rng(77)
    rows = rng.standard_normal((50_000, 288)).astype(np.float32)
    q = rng.standard_normal((2, 288)).astype(np.float32)
    bank = CudaMLARouteSidecar.build().create_bank(rows)
    try:
        mapped, rec = bank.route_topk(q, topk=3, warmup=1, route_repeats=2)
    finally:
        bank.close()
    want, _, _ = oracle.mla_route(rows, q, 3)
    np.testing.assert_array_equal(mapped, want)
    assert all(t > 0.0 for t in rec.device_route_ms_runs)
