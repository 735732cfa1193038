"""The allocation-free MLA route (grm_mla_hip_route_noalloc) against the
allocating one (grm_mla_hip_route), both called through the C ABI.

Bar: ids and score bits equal on every query, on two calls in a row, the
second on a smaller bank with fewer grid blocks and a smaller topk, so a
stale list the first call left in the shared scratch array would show.
The outputs also match the oracle (the allocating route's own bar).
A two-thread case routes two banks on one GPU at the same time, many
times over, and every answer must equal the oracle's.
"""

import threading

import numpy as np
import pytest

import oracle
from graftrepository_amd import MlaNodeBank, workloads as wl
from graftrepository_amd.node_bank import as_bf16_bits, bf16_bits_to_f32
from graftrepository_amd.payload import DeviceArray

pytestmark = pytest.mark.gpu
NO_ID = np.iinfo(np.uint64).max
F32, BF16 = 0, 1

def route_both(lib, bank, queries, dtype_code, topk):
    """(ids, scores) from the allocation-free route and from the allocating
    route with the same device-resident queries."""
    q_count = queries.shape[0]
    with DeviceArray.from_host(queries) as dq, \
            DeviceArray((q_count, topk), np.uint64) as d_ids, \
            DeviceArray((q_count, topk), np.float32) as d_sc:
        rc = lib.grm_mla_hip_route_noalloc(bank._h, dq.ptr, dtype_code, q_count, bank.dim,
                                           topk, d_ids.ptr, d_sc.ptr)
        assert rc == 0, lib.grm_hip_last_error()
        got = (d_ids.to_host(), d_sc.to_host())
        ids = np.empty((q_count, topk), dtype=np.uint64)
        sc = np.empty((q_count, topk), dtype=np.float32)
        rc = lib.grm_mla_hip_route(bank._h, dq.ptr, dtype_code, 1, q_count, bank.dim, 0, topk,
                                   ids.ctypes.data, sc.ctypes.data, None)
        assert rc == 0, lib.grm_hip_last_error()
    return got, (ids, sc)

def assert_same(a, b):
    np.testing.assert_array_equal(a[0], b[0])
    filled = b[0] != NO_ID
    assert np.all(np.isnan(a[1][~filled])) and np.all(np.isnan(b[1][~filled]))
    np.testing.assert_array_equal(a[1][filled].view(np.uint32), b[1][filled].view(np.uint32))

def test_noalloc_matches_allocating_route_twice(hip_lib):
    lib = hip_lib
    # call 1: 300k x 288 fp32, 3 queries, top-16 (the pipelined kernel, one
    # block per CU); one NaN row and a duplicated row make a tie block
    rows = wl.mla_rows(300_000, 288, seed=71)
    rows[1234] = np.nan
    rows[5000] = rows[77]
    ids1 = np.arange(300_000, dtype=np.uint64)[::-1].copy() + 9
    qs = wl.mla_queries(3, 288, seed=71)
    qs[2] = rows[77]
    with MlaNodeBank(rows, ids1) as bank:
        got, want = route_both(lib, bank, qs, F32, 16)
    assert_same(got, want)
    o_ids, o_sc, _ = oracle.mla_route(rows, qs, 16, node_ids=ids1)
    assert_same(got, (o_ids, o_sc))

    # call 2, smaller: 700 x 61 bf16, 2 bf16 queries, top-5 (the plain
    # kernel, a handful of blocks), one NaN query (no results)
    rng = np.random.default_rng(72)
    rows2 = as_bf16_bits(rng.standard_normal((700, 61)).astype(np.float32))
    qs2 = as_bf16_bits(rng.standard_normal((2, 61)).astype(np.float32))
    qs2[1, 5] = 0x7FC0  # bf16 NaN
    with MlaNodeBank(rows2, dtype="bf16") as bank:
        got2, want2 = route_both(lib, bank, qs2, BF16, 5)
    assert_same(got2, want2)
    assert np.all(got2[0][1] == NO_ID)
    o_ids2, o_sc2, _ = oracle.mla_route(bf16_bits_to_f32(rows2), bf16_bits_to_f32(qs2), 5)
    assert_same(got2, (o_ids2, o_sc2))

def test_noalloc_rejects_bad_arguments(hip_lib):
    lib = hip_lib
    rows = wl.mla_rows(100, 32, seed=73)
    with MlaNodeBank(rows) as bank, DeviceArray((1, 32), np.float32) as dq, \
            DeviceArray((1, 16), np.uint64) as d_ids:
        # topk above the live count, a wrong dim, a null output
        assert lib.grm_mla_hip_route_noalloc(bank._h, dq.ptr, F32, 1, 32, 17, d_ids.ptr,
                                             None) == -1
        assert lib.grm_mla_hip_route_noalloc(bank._h, dq.ptr, F32, 1, 31, 3, d_ids.ptr,
                                             None) == -1
        assert lib.grm_mla_hip_route_noalloc(bank._h, dq.ptr, F32, 1, 32, 3, None, None) == -1
        assert b"null" in lib.grm_hip_last_error()

def test_noalloc_two_threads_two_banks(hip_lib):
    """Two host threads, each routing its own bank on the same GPU through
    the allocation-free entry, start together and call it repeatedly (ctypes
    releases the GIL, so the calls overlap on the host).  Every result must
    equal the oracle's ids and score bits."""
    lib = hip_lib
    rows_a = wl.mla_rows(200_000, 288, seed=81)
    qs_a = wl.mla_queries(2, 288, seed=81)
    rows_b = wl.mla_rows(120_000, 128, seed=82)
    qs_b = wl.mla_queries(3, 128, seed=82)
    want_a = oracle.mla_route(rows_a, qs_a, 8)[:2]
    want_b = oracle.mla_route(rows_b, qs_b, 5)[:2]
    reps = 40
    start = threading.Barrier(2)
    errors: list = []
    results: dict = {}

    def worker(name, bank, qs, topk):
        try:
            q_count = qs.shape[0]
            outs = []
            with DeviceArray.from_host(qs) as dq, \
                    DeviceArray((q_count, topk), np.uint64) as d_ids, \
                    DeviceArray((q_count, topk), np.float32) as d_sc:
                start.wait(timeout=60)
                for _ in range(reps):
                    rc = lib.grm_mla_hip_route_noalloc(bank._h, dq.ptr, F32, q_count, bank.dim,
                                                       topk, d_ids.ptr, d_sc.ptr)
                    if rc != 0:
                        raise RuntimeError(f"rc {rc}: {lib.grm_hip_last_error()}")
                    outs.append((d_ids.to_host(), d_sc.to_host()))
            results[name] = outs
        except BaseException as exc:  # reported by the main thread
            errors.append((name, exc))
            start.abort()

    with MlaNodeBank(rows_a) as bank_a, MlaNodeBank(rows_b) as bank_b:
        threads = [threading.Thread(target=worker, args=("a", bank_a, qs_a, 8)),
                   threading.Thread(target=worker, args=("b", bank_b, qs_b, 5))]
        for t in threads:
            t.start()
        for t in threads:
            t.join(timeout=120)
        assert not any(t.is_alive() for t in threads), "a routing thread did not finish"
    assert not errors, errors
    assert len(results["a"]) == reps and len(results["b"]) == reps
    for got in results["a"]:
        assert_same(got, want_a)
    for got in results["b"]:
        assert_same(got, want_b)
