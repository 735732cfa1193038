"""MLA route parity on the GPU: the HIP library against the fp64 oracle.

Bar: node ids bit-exact (ties to the lowest node id) and scores bit-exact
(the kernel evaluates the reference's fp64 law in the reference's order,
cpp/grm_runtime.cpp:3518-3545).  Cases follow the reference's gates and
tests: orthonormal / duplicate-row tie blocks and NaN rows
(scripts/grm_mla_cuda_route_gate.py:73-86), NaN query -> unfilled slots
(core/grm_cuda_router.py:460-475), row ids through the sidecar surface.
"""

import numpy as np
import pytest

import oracle
from graftrepository_amd import MlaNodeBank, workloads as wl
from graftrepository_amd.grm_hip_router import CudaMLARouteSidecar
from graftrepository_amd.mla_probe import HipProbe
from graftrepository_amd.node_bank import bf16_bits_to_f32

pytestmark = pytest.mark.gpu
NO_ID = np.iinfo(np.uint64).max


def assert_same(res_ids, res_scores, want_ids, want_scores):
    np.testing.assert_array_equal(res_ids, want_ids)
    filled = want_ids != NO_ID
    assert np.all(np.isnan(res_scores[~filled]))
    np.testing.assert_array_equal(res_scores[filled].view(np.uint32),
                                  want_scores[filled].view(np.uint32))


def test_small_config_parity(hip_lib):
    rows = wl.mla_rows(10_000, 288, seed=11)
    qs = wl.mla_queries(16, 288, seed=11)
    with MlaNodeBank(rows) as bank:
        for k in (1, 3, 16):
            res = bank.route(qs, k)
            ids, sc, _ = oracle.mla_route(rows, qs, k)
            assert_same(res.ids, res.scores, ids, sc)


def test_small_config_against_python_numpy_law(hip_lib):
    """The 10,000 x 288 workload against the reference's Python route
    (numpy fp32 dot, stable sort; core/graft_arena.py:733-801): ids equal
    wherever the fp32 dot's rounding bound cannot reorder the top k,
    scores within 1e-5 relative."""
    d, k = 288, 3
    rows = wl.mla_rows(10_000, d, seed=1)
    qs = wl.mla_queries(32, d, seed=1)
    gamma = d * 2.0 ** -24 / (1 - d * 2.0 ** -24)
    with MlaNodeBank(rows) as bank:
        res = bank.route(qs, k)
    ids_np, sc_np, _ = oracle.mla_route_numpy(rows, qs, k + 1)
    absdot = np.abs(rows.astype(np.float64)) @ np.abs(qs.astype(np.float64)).T
    compared = 0
    for j in range(qs.shape[0]):
        assert np.allclose(res.scores[j], sc_np[j, :k], rtol=1e-5, atol=0)
        gaps = -np.diff(sc_np[j].astype(np.float64))
        if np.all(gaps > 2 * gamma * absdot[:, j].max()):
            assert res.ids[j].astype(np.int64).tolist() == ids_np[j, :k].tolist()
            compared += 1
    assert compared >= qs.shape[0] // 2


@pytest.mark.parametrize("dim", [1, 3, 4, 5, 64, 127, 128, 256, 288, 300, 1000])
def test_dims_and_ragged_tiles(hip_lib, dim):
    rng = np.random.default_rng(dim)
    n = 777
    rows = rng.standard_normal((n, dim)).astype(np.float32)
    qs = rng.standard_normal((3, dim)).astype(np.float32)
    with MlaNodeBank(rows) as bank:
        res = bank.route(qs, 7)
    ids, sc, _ = oracle.mla_route(rows, qs, 7)
    assert_same(res.ids, res.scores, ids, sc)


def test_duplicate_rows_tie_to_lowest_node_id(hip_lib):
    rng = np.random.default_rng(5)
    base = rng.standard_normal((40, 64)).astype(np.float32)
    rows = np.repeat(base, 25, axis=0)           # 1000 rows, 25-way tie blocks
    node_ids = rng.permutation(1000).astype(np.uint64) + 1000
    q = base[7] + np.float32(0.25) * base[3]
    with MlaNodeBank(rows, node_ids) as bank:
        res = bank.route(q, 16)
    ids, sc, _ = oracle.mla_route(rows, q, 16, node_ids=node_ids)
    assert_same(res.ids, res.scores, ids, sc)
    top_block = node_ids[7 * 25:8 * 25]
    assert list(res.ids[0]) == sorted(top_block.tolist())[:16]


def test_orthonormal_closed_form(hip_lib):
    dim = 128
    rows = np.eye(dim, dtype=np.float32)
    q = np.zeros(dim, dtype=np.float32)
    q[[5, 9, 77]] = [3.0, 2.0, 1.0]
    with MlaNodeBank(rows) as bank:
        res = bank.route(q, 3)
    assert res.ids[0].tolist() == [5, 9, 77]
    qn = np.sqrt(14.0)
    want = [np.float32(v / (qn * 1.0 + 1e-8)) for v in (3.0, 2.0, 1.0)]
    np.testing.assert_array_equal(res.scores[0], np.asarray(want, np.float32))


def test_nan_rows_dropped_and_nan_query_unfilled(hip_lib):
    rng = np.random.default_rng(9)
    rows = rng.standard_normal((300, 48)).astype(np.float32)
    rows[[0, 17, 299], 3] = np.nan
    rows[42, 0] = np.inf
    qs = rng.standard_normal((2, 48)).astype(np.float32)
    with MlaNodeBank(rows) as bank:
        res = bank.route(qs, 10)
        ids, sc, _ = oracle.mla_route(rows, qs, 10)
        assert_same(res.ids, res.scores, ids, sc)
        assert not set(res.ids.ravel().tolist()) & {0, 17, 42, 299}
        bad = qs[:1].copy()
        bad[0, 5] = np.nan
        res = bank.route(bad, 4)
        assert np.all(res.ids == NO_ID)
    # reference hand case: tests/test_grm_router_baseline.py:26-33
    routes = np.asarray([[np.nan, 0.0], [1.0, 0.0], [0.0, 1.0]], np.float32)
    with MlaNodeBank(routes) as bank:
        res = bank.route(np.asarray([1.0, 0.0], np.float32), 2)
    assert res.ids[0].tolist() == [1, 2]


def test_bf16_bank_parity(hip_lib):
    rows = wl.mla_rows(5000, 288, seed=21, dtype="bf16")
    qs = wl.mla_queries(8, 288, seed=21, dtype="bf16")
    with MlaNodeBank(rows, dtype="bf16") as bank:
        res = bank.route(qs, 8)
    ids, sc, _ = oracle.mla_route(bf16_bits_to_f32(rows).reshape(rows.shape),
                                  bf16_bits_to_f32(qs).reshape(qs.shape), 8)
    assert_same(res.ids, res.scores, ids, sc)


def test_append_evict_matches_oracle_on_live_set(hip_lib):
    rng = np.random.default_rng(33)
    dim = 96
    rows = rng.standard_normal((1000, dim)).astype(np.float32)
    ids0 = np.arange(1000, dtype=np.uint64) * 3
    qs = rng.standard_normal((4, dim)).astype(np.float32)
    with MlaNodeBank(rows, ids0, capacity=1500) as bank:
        live = {int(i): rows[j] for j, i in enumerate(ids0)}
        for step in range(4):
            ev = rng.choice(sorted(live), size=60, replace=False).astype(np.uint64)
            bank.evict(ev)
            for i in ev.tolist():
                del live[i]
            new_ids = np.arange(60, dtype=np.uint64) + 10_000 + step * 100
            new_rows = rng.standard_normal((60, dim)).astype(np.float32)
            bank.append(new_rows, new_ids)
            for i, r in zip(new_ids.tolist(), new_rows):
                live[i] = r
            res = bank.route(qs, 9)
            keys = np.asarray(sorted(live), dtype=np.uint64)
            mat = np.stack([live[int(k)] for k in keys])
            want, wsc, _ = oracle.mla_route(mat, qs, 9, node_ids=keys)
            assert_same(res.ids, res.scores, want, wsc)
        info = bank.info()
        assert info["live"] == len(live)
        with pytest.raises(RuntimeError):
            bank.evict([123456789])
        with pytest.raises(RuntimeError):
            bank.append(rows[:1], [int(keys[0])])


def test_reference_surface_row_ids_and_device_entry(hip_lib):
    rows = wl.mla_rows(2000, 128, seed=44)
    qs = wl.mla_queries(6, 128, seed=44)
    node_ids = np.arange(2000, dtype=np.uint64) + 500
    sidecar = CudaMLARouteSidecar.build()
    bank = sidecar.create_bank(rows, node_ids)
    mapped, receipt = bank.route_topk(qs, topk=5, warmup=2)
    want, _, _ = oracle.mla_route(rows, qs, 5)
    np.testing.assert_array_equal(mapped, node_ids[want])
    assert receipt.measured_queries == 4
    probe = HipProbe()
    dq = probe.upload_queries(qs)
    mapped_d, _ = bank.route_topk_device(dq, topk=5)
    np.testing.assert_array_equal(mapped_d, mapped)
    dq.close()
    one_shot, _, _ = probe.route_topk(rows, qs, warmup=0, topk=5)
    np.testing.assert_array_equal(one_shot, want)
    bank.close()
    with pytest.raises(RuntimeError):
        bank.route_topk(qs, topk=5)


def test_invalid_arguments_rejected(hip_lib):
    rows = wl.mla_rows(100, 16, seed=1)
    with MlaNodeBank(rows) as bank:
        for k in (0, 17, 101):
            with pytest.raises(RuntimeError):
                bank.route(rows[:1], k)
        with pytest.raises(RuntimeError):
            bank.route(rows[:2], 3, warmup=2)
    arena = HipProbe().create_arena(rows)
    with pytest.raises(ValueError):
        arena.route_topk(rows[:1, :8], warmup=0, topk=1)


def test_repeated_calls_are_stable(hip_lib):
    rows = wl.mla_rows(200_000, 288, seed=55)
    qs = wl.mla_queries(3, 288, seed=55)
    ids, sc, _ = oracle.mla_route(rows, qs, 5)
    with MlaNodeBank(rows) as bank:
        for _ in range(40):
            res = bank.route(qs, 5)
            assert_same(res.ids, res.scores, ids, sc)


def test_headline_size_parity(hip_lib):
    cfg = wl.MLA_HEADLINE
    rows = wl.mla_rows(cfg["nodes"], cfg["dim"], seed=cfg["seed"])
    qs = wl.mla_queries(3, cfg["dim"], seed=cfg["seed"])
    with MlaNodeBank(rows) as bank:
        res = bank.route(qs, cfg["topk"])
    ids, sc, _ = oracle.mla_route(rows, qs, cfg["topk"])
    assert_same(res.ids, res.scores, ids, sc)


# ------------------------------------------------ batched route (bf16 banks)

def _f32(bits):
    return bf16_bits_to_f32(bits).reshape(bits.shape)


@pytest.mark.parametrize("nq,k", [(4, 1), (33, 8), (64, 16), (256, 8), (300, 5)])
def test_batched_bf16_route_matches_oracle(hip_lib, nq, k):
    rows = wl.mla_rows(40_000, 288, seed=61, dtype="bf16")
    qs = wl.mla_queries(nq, 288, seed=61, dtype="bf16")
    with MlaNodeBank(rows, dtype="bf16") as bank:
        res = bank.route(qs, k)
        stats = bank.route_stats()
    ids, sc, _ = oracle.mla_route(_f32(rows), _f32(qs), k)
    assert_same(res.ids, res.scores, ids, sc)
    assert stats["batched"] == nq and stats["fallbacks"] <= max(1, nq // 50)


@pytest.mark.parametrize("dim", [16, 100, 128, 200, 256, 288])
def test_batched_dims(hip_lib, dim):
    rows = wl.mla_rows(3000, dim, seed=dim, dtype="bf16")
    qs = wl.mla_queries(40, dim, seed=dim, dtype="bf16")
    with MlaNodeBank(rows, dtype="bf16") as bank:
        res = bank.route(qs, 6, warmup=3)
        stats = bank.route_stats()
    ids, sc, _ = oracle.mla_route(_f32(rows), _f32(qs), 6)
    assert_same(res.ids, res.scores, ids, sc)
    assert stats["batched"] == 40


def test_batched_ties_zero_and_nan_rows(hip_lib):
    # Duplicate rows tie exactly (lowest node id first, possibly through
    # the single-query path when no certificate exists), an all-zero row
    # scores 0, NaN rows and a NaN query are never ranked.
    rng = np.random.default_rng(62)
    base = rng.standard_normal((60, 128)).astype(np.float32)
    rows = np.repeat(base, 20, axis=0)
    rows[5] = 0.0
    rows[17, 3] = np.nan
    node_ids = rng.permutation(rows.shape[0]).astype(np.uint64) + 7
    qs = np.concatenate([base[:12] + 0.1 * base[12:24],
                         np.zeros((1, 128), np.float32)])
    qs[3, 0] = np.nan
    bits, qbits = oracle.bf16_bits(rows), oracle.bf16_bits(qs)
    with MlaNodeBank(bits, node_ids, dtype="bf16") as bank:
        res = bank.route(qbits, 10)
    ids, sc, _ = oracle.mla_route(_f32(bits), _f32(qbits), 10, node_ids=node_ids)
    assert_same(res.ids, res.scores, ids, sc)


def test_batched_negative_tops_huge_rows_and_infinities(hip_lib):
    # Where the screen cannot certify, the single-query path answers:
    # every score negative (a non-positive threshold), a query whose
    # products with the largest row could overflow fp32, and rows holding
    # an infinity (the law scores them NaN) beside ordinary rows.
    rng = np.random.default_rng(65)
    rows = np.abs(rng.standard_normal((3000, 64))).astype(np.float32)
    qs = -np.abs(rng.standard_normal((8, 64))).astype(np.float32)
    bits, qbits = oracle.bf16_bits(rows), oracle.bf16_bits(qs)
    with MlaNodeBank(bits, dtype="bf16") as bank:
        res = bank.route(qbits, 6)
    ids, sc, _ = oracle.mla_route(_f32(bits), _f32(qbits), 6)
    assert_same(res.ids, res.scores, ids, sc)

    rows = rng.standard_normal((3000, 64)).astype(np.float32)
    rows[7] *= np.float32(1e30)
    rows[9, 2] = np.inf
    rows[11, 5] = -np.inf
    qs = rng.standard_normal((8, 64)).astype(np.float32)
    qs[0] *= np.float32(1e10)
    qs[1] = rows[7] / np.float32(1e30)
    bits, qbits = oracle.bf16_bits(rows), oracle.bf16_bits(qs)
    with MlaNodeBank(bits, dtype="bf16") as bank:
        res = bank.route(qbits, 6)
    ids, sc, _ = oracle.mla_route(_f32(bits), _f32(qbits), 6)
    assert_same(res.ids, res.scores, ids, sc)
    assert not {9, 11} & set(res.ids.ravel().tolist())


def test_batched_f32_queries_on_bf16_bank(hip_lib):
    # fp32 queries are rounded to bf16 for the matrix cores; the bound
    # covers the rounding and the law uses the fp32 values.
    rows = wl.mla_rows(20_000, 288, seed=63, dtype="bf16")
    qs = wl.mla_queries(16, 288, seed=63)
    with MlaNodeBank(rows, dtype="bf16") as bank:
        res = bank.route(qs, 5, query_dtype="f32")
    ids, sc, _ = oracle.mla_route(_f32(rows), qs, 5)
    assert_same(res.ids, res.scores, ids, sc)


def test_batched_after_append_and_evict(hip_lib):
    rng = np.random.default_rng(64)
    rows = wl.mla_rows(5000, 256, seed=64, dtype="bf16")
    ids0 = np.arange(5000, dtype=np.uint64) * 2 + 1
    qs = wl.mla_queries(24, 256, seed=64, dtype="bf16")
    live = {int(i): rows[j] for j, i in enumerate(ids0)}
    with MlaNodeBank(rows, ids0, dtype="bf16", capacity=6000) as bank:
        for step in range(3):
            ev = rng.choice(sorted(live), size=300, replace=False).astype(np.uint64)
            bank.evict(ev)
            for i in ev.tolist():
                del live[i]
            new = wl.mla_rows(250, 256, seed=640 + step, dtype="bf16")
            nid = np.arange(250, dtype=np.uint64) + 100_000 + 1000 * step
            bank.append(new, nid)
            live.update({int(i): r for i, r in zip(nid.tolist(), new)})
            res = bank.route(qs, 8)
            keys = np.asarray(sorted(live), dtype=np.uint64)
            mat = np.stack([live[int(k)] for k in keys])
            want, wsc, _ = oracle.mla_route(_f32(mat), _f32(qs), 8, node_ids=keys)
            assert_same(res.ids, res.scores, want, wsc)


def test_batched_config_parity(hip_lib):
    # 256 queries x 1,000,000 x 288 bf16, top-8: one screen pass
    cfg = wl.MLA_BATCHED
    rows = wl.mla_rows(cfg["nodes"], cfg["dim"], seed=cfg["seed"], dtype="bf16")
    qs = wl.mla_queries(cfg["queries"], cfg["dim"], seed=cfg["seed"], dtype="bf16")
    with MlaNodeBank(rows, dtype="bf16") as bank:
        res = bank.route(qs, cfg["topk"])
        stats = bank.route_stats()
    ids, sc, _ = oracle.mla_route(_f32(rows), _f32(qs), cfg["topk"])
    assert_same(res.ids, res.scores, ids, sc)
    assert stats["passes"] == 1 and stats["fallbacks"] <= 2


@pytest.mark.parametrize("dim", [100, 256, 288])  # K-steps 8, 16 and 18
def test_batched_ring_screen_dims_and_churn(hip_lib, dim):
    # Passes of more than 128 queries run the ring screen (queries in
    # registers, the bank streamed through LDS); its slot weights follow
    # the bank through evictions and appends.  Ids and score bits against
    # the oracle, before and after each churn round.
    rng = np.random.default_rng(dim + 70)
    rows = wl.mla_rows(30_000, dim, seed=dim + 7, dtype="bf16")
    ids0 = np.arange(30_000, dtype=np.uint64) * 3 + 5
    qs = wl.mla_queries(200, dim, seed=dim + 7, dtype="bf16")
    live = {int(i): rows[j] for j, i in enumerate(ids0)}
    with MlaNodeBank(rows, ids0, dtype="bf16", capacity=32_000) as bank:
        for step in range(3):
            res = bank.route(qs, 8)
            keys = np.asarray(sorted(live), dtype=np.uint64)
            mat = np.stack([live[int(k)] for k in keys])
            want, wsc, _ = oracle.mla_route(_f32(mat), _f32(qs), 8, node_ids=keys)
            assert_same(res.ids, res.scores, want, wsc)
            ev = rng.choice(keys, size=900, replace=False)
            bank.evict(ev)
            for i in ev.tolist():
                del live[i]
            new = wl.mla_rows(800, dim, seed=dim * 10 + step, dtype="bf16")
            nid = np.arange(800, dtype=np.uint64) + 1_000_000 + 10_000 * step
            bank.append(new, nid)
            live.update({int(i): r for i, r in zip(nid.tolist(), new)})
        stats = bank.route_stats()
    assert stats["batched"] == 600 and stats["fallbacks"] <= 6


@pytest.mark.parametrize("count", [48, 256])  # 256: the full-pass screen
def test_batched_copies_of_best_rows_far_apart(hip_lib, count):
    # Exact copies of the best rows sit in different screen sub-streams
    # (slots 50.. and 100,000..), so the merge sees tied candidates from
    # two wavefronts; NaN and zero rows share tiles with the copies.
    n, dim = 140_000, 288
    rows = wl.mla_rows(n, dim, seed=65, dtype="bf16")
    qs = wl.mla_queries(count, dim, seed=65, dtype="bf16")
    rows[100_000:100_004] = qs[:4]          # near-perfect matches
    rows[50:54] = qs[:4]                    # their copies, far from them
    rows[1000] = qs[5]
    rows[7] = oracle.bf16_bits(np.full(dim, np.nan, np.float32))
    rows[8] = 0
    node_ids = np.arange(n, dtype=np.uint64)[::-1].copy()
    with MlaNodeBank(rows, node_ids, dtype="bf16") as bank:
        res = bank.route(qs, 8)
        stats = bank.route_stats()
    ids, sc, _ = oracle.mla_route(_f32(rows), _f32(qs), 8, node_ids=node_ids)
    assert_same(res.ids, res.scores, ids, sc)
    assert stats["batched"] == count


@pytest.mark.parametrize("dim,dtype", [(288, "f32"), (96, "f32"), (256, "bf16")])
def test_untimed_routes_wait_on_completion_flags(hip_lib, dim, dtype):
    # Routes that ask for no device time wait on the route blocks'
    # completion flags instead of a stream event: the same results as timed
    # routes, for the pipelined kernel (288 values), the plain kernel (96),
    # several queries with warmup, batched bf16 queries, and across bank
    # changes.
    rng = np.random.default_rng(dim)
    rows = wl.mla_rows(120_000, dim, seed=dim, dtype=dtype)
    ids0 = np.arange(120_000, dtype=np.uint64) * 5 + 2
    qs = wl.mla_queries(24, dim, seed=dim + 1, dtype=dtype)
    f = _f32 if dtype == "bf16" else (lambda x: x)
    live = np.ones(120_000, bool)
    with MlaNodeBank(rows, ids0, dtype=dtype) as bank:
        for step in range(2):
            for n, warm in ((1, 0), (3, 1), (24, 0)):
                want, wsc, _ = oracle.mla_route(f(rows[live]), f(qs[:n]), 7, node_ids=ids0[live])
                for timed in (False, True, False):
                    r = bank.route(qs[:n], 7, warmup=warm, timed=timed)
                    assert_same(r.ids, r.scores, want, wsc)
                    assert np.isnan(r.device_ms) != timed
            ev = rng.choice(np.flatnonzero(live), size=500, replace=False)
            bank.evict(ids0[ev])
            live[ev] = False
