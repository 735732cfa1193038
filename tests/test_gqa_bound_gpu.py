"""Bound-and-verify GQA route (batched queries) on the GPU against the oracle.

Routes with more than 24 query columns per kv head (batched queries, or
queries of many tokens, whose columns are screened in passes of 64) screen
every node once per pass, bound each node's score, and evaluate the law
exactly on the nodes whose bound reaches the k-th best lower bound.  GRM_HIP_GQA_BOUND=1 forces that
path for any batch and 0 disables it; both must give the oracle's ids and
score bits (cpp/grm_runtime.cpp:2980-3029 gqa_raw_score, ties to the lowest
node id per cpp/grm_runtime.cpp:75-82).
"""

import numpy as np
import pytest

import oracle
from graftrepository_amd import GqaNodeBank, workloads as wl
from graftrepository_amd.node_bank import bf16_bits_to_f32

pytestmark = pytest.mark.gpu
NO_ID = np.iinfo(np.uint64).max


def assert_same(res, want_ids, want_scores):
    np.testing.assert_array_equal(res.ids, want_ids)
    filled = want_ids != NO_ID
    assert np.all(np.isnan(res.scores[~filled]))
    np.testing.assert_array_equal(res.scores[filled].view(np.uint32),
                                  want_scores[filled].view(np.uint32))


def ragged(rng, n, kv, hd, lo, hi):
    lens = rng.integers(lo, hi + 1, size=n).astype(np.uint64)
    offs = np.zeros(n + 1, np.uint64)
    offs[1:] = np.cumsum(lens)
    keys = rng.standard_normal(int(offs[-1]) * kv * hd).astype(np.float32)
    return keys, offs


@pytest.fixture(params=["1", "auto"])
def bound_mode(request, monkeypatch):
    if request.param == "auto":
        monkeypatch.delenv("GRM_HIP_GQA_BOUND", raising=False)
    else:
        monkeypatch.setenv("GRM_HIP_GQA_BOUND", request.param)
    return request.param


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_half_banks_batched(hip_lib, bound_mode, dtype):
    # nodes up to 600 tokens: several work items per node
    lens = wl.gqa_lengths(500, seed=101, lo=1, hi=600)
    keys, offs = wl.gqa_bank(lens, 8, 128, seed=101, dtype=dtype)
    qs = wl.gqa_queries(16, 32, 1, 128, seed=101, dtype="bf16")
    with GqaNodeBank(keys, offs, kv_heads=8, head_dim=128, dtype=dtype) as bank:
        res = bank.route(qs, 6, query_dtype="bf16")
    code = oracle.BF16 if dtype == "bf16" else oracle.F16
    ids, sc, _ = oracle.gqa_route(keys, code, offs, 8, 128,
                                  bf16_bits_to_f32(qs).reshape(qs.shape), 6)
    assert_same(res, ids, sc)


@pytest.mark.parametrize("group,scale_dtype", [(128, "f16"), (128, "f32"),
                                               (32, "f32"), (64, "f16")])
def test_int8_batched(hip_lib, bound_mode, group, scale_dtype):
    # group == head_dim takes the factored-scale screen, smaller groups the
    # per-element dequantisation
    rng = np.random.default_rng(group + (1 if scale_dtype == "f16" else 0))
    keys, offs = ragged(rng, 400, 8, 128, 1, 500)
    codes, scales = oracle.quantize_int8(keys.reshape(-1, 128), group, scale_dtype)
    qs = rng.standard_normal((16, 32, 1, 128)).astype(np.float32)
    with GqaNodeBank(codes, offs, kv_heads=8, head_dim=128, dtype="i8",
                     scales=scales, scale_dtype=scale_dtype, group_size=group) as bank:
        res = bank.route(qs, 5)
    ids, sc, _ = oracle.gqa_route(codes, oracle.I8, offs, 8, 128, qs, 5,
                                  scales=scales, scale_dtype=scale_dtype,
                                  group_size=group)
    assert_same(res, ids, sc)


@pytest.mark.parametrize("hd", [64, 256])
def test_int8_head_dims(hip_lib, bound_mode, hd):
    rng = np.random.default_rng(hd)
    keys, offs = ragged(rng, 150, 4, hd, 1, 300)
    codes, scales = oracle.quantize_int8(keys.reshape(-1, hd), hd, "f16")
    qs = rng.standard_normal((8, 16, 2, hd)).astype(np.float32)  # 8*4*2 = 64 columns
    with GqaNodeBank(codes, offs, kv_heads=4, head_dim=hd, dtype="i8",
                     scales=scales, scale_dtype="f16", group_size=hd) as bank:
        res = bank.route(qs, 4)
    ids, sc, _ = oracle.gqa_route(codes, oracle.I8, offs, 4, hd, qs, 4,
                                  scales=scales, scale_dtype="f16", group_size=hd)
    assert_same(res, ids, sc)


@pytest.mark.parametrize("Qt,nq", [(4, 4), (2, 5), (1, 1)])
def test_query_tokens_and_small_batches(hip_lib, bound_mode, Qt, nq):
    lens = wl.gqa_lengths(300, seed=111, lo=1, hi=400)
    keys, offs = wl.gqa_bank(lens, 8, 128, seed=111, dtype="bf16")
    qs = wl.gqa_queries(nq, 32, Qt, 128, seed=111, dtype="f32")
    with GqaNodeBank(keys, offs, kv_heads=8, head_dim=128, dtype="bf16") as bank:
        res = bank.route(qs, 7)
    ids, sc, _ = oracle.gqa_route(keys, oracle.BF16, offs, 8, 128, qs, 7)
    assert_same(res, ids, sc)


def test_many_passes_with_warmup(hip_lib, bound_mode):
    # 40 queries: passes of 16, 16 and 8 (the last one is small enough for
    # the screen-and-refine path unless the bound path is forced)
    lens = wl.gqa_lengths(250, seed=121, lo=1, hi=300)
    keys, offs = wl.gqa_bank(lens, 8, 64, seed=121, dtype="f16")
    qs = wl.gqa_queries(40, 32, 1, 64, seed=121, dtype="bf16")
    with GqaNodeBank(keys, offs, kv_heads=8, head_dim=64, dtype="f16") as bank:
        res = bank.route(qs, 3, query_dtype="bf16", warmup=5)
    ids, sc, _ = oracle.gqa_route(keys, oracle.F16, offs, 8, 64,
                                  bf16_bits_to_f32(qs).reshape(qs.shape), 3)
    assert_same(res, ids, sc)


def test_ties_make_every_tied_node_a_candidate(hip_lib, bound_mode):
    # 120 identical nodes: their bounds coincide, all of them are candidates,
    # and the exact scores tie, so the order falls to the node ids.
    rng = np.random.default_rng(131)
    block = rng.standard_normal(8 * 70 * 128).astype(np.float32)
    others = rng.standard_normal(8 * 70 * 128 * 30).astype(np.float32) * 0.5
    keys = oracle.bf16_bits(np.concatenate([np.tile(block, 120), others]))
    offs = np.arange(151, dtype=np.uint64) * 70
    ids = (np.arange(150, dtype=np.uint64)[::-1] * 3 + 11).copy()
    qs = rng.standard_normal((16, 32, 1, 128)).astype(np.float32)
    with GqaNodeBank(keys, offs, kv_heads=8, head_dim=128, dtype="bf16",
                     node_ids=ids) as bank:
        res = bank.route(qs, 16)
    want, wsc, _ = oracle.gqa_route(keys, oracle.BF16, offs, 8, 128, qs, 16,
                                    node_ids=ids)
    assert_same(res, want, wsc)


def test_empty_nodes_nonfinite_keys_and_bad_query(hip_lib, bound_mode):
    rng = np.random.default_rng(141)
    kv, hd, H = 4, 128, 16
    lens = rng.integers(1, 90, size=120).astype(np.uint64)
    lens[[3, 17, 40]] = 0
    offs = np.zeros(lens.size + 1, np.uint64)
    offs[1:] = np.cumsum(lens)
    keys = rng.standard_normal(int(offs[-1]) * kv * hd).astype(np.float32) * 0.01
    for node in (5, 60):  # poison two nodes
        keys[int(offs[node]) * kv * hd + 11] = np.nan
    bits = oracle.f16_bits(keys)
    qs = rng.standard_normal((16, H, 1, hd)).astype(np.float32)
    qs[9, 2, 0, 3] = np.inf
    with GqaNodeBank(bits, offs, kv_heads=kv, head_dim=hd, dtype="f16") as bank:
        res = bank.route(qs, 6)
    ids, sc, _ = oracle.gqa_route(bits, oracle.F16, offs, kv, hd, qs, 6)
    assert_same(res, ids, sc)
    assert not {5, 60} & set(res.ids.reshape(-1).tolist())
    assert sorted(res.ids[9][:3].tolist()) == [3, 17, 40]  # only empty nodes score


def test_after_evict_append_compact(hip_lib, bound_mode):
    rng = np.random.default_rng(151)
    kv, hd, H = 8, 128, 32
    keys, offs = ragged(rng, 200, kv, hd, 1, 300)
    codes, scales = oracle.quantize_int8(keys.reshape(-1, hd), hd, "f16")
    codes, scales = codes.reshape(-1), scales.reshape(-1)
    ids0 = np.arange(200, dtype=np.uint64) + 1
    per = [(codes[int(offs[j]) * kv * hd:int(offs[j + 1]) * kv * hd],
            scales[int(offs[j]) * kv:int(offs[j + 1]) * kv]) for j in range(200)]
    blocks = dict(zip(ids0.tolist(), per))
    qs = rng.standard_normal((16, H, 1, hd)).astype(np.float32)
    with GqaNodeBank(codes, offs, kv_heads=kv, head_dim=hd, dtype="i8", scales=scales,
                     scale_dtype="f16", group_size=hd, node_ids=ids0,
                     capacity_nodes=300, capacity_tokens=200_000) as bank:
        for step in range(3):
            ev = rng.choice(sorted(blocks), size=20, replace=False)
            bank.evict(ev)
            for i in ev.tolist():
                del blocks[i]
            nk, no = ragged(rng, 15, kv, hd, 0, 300)
            nc, ns = oracle.quantize_int8(nk.reshape(-1, hd), hd, "f16")
            nc, ns = nc.reshape(-1), ns.reshape(-1)
            nl = np.diff(no).astype(np.uint64)
            nid = np.arange(15, dtype=np.uint64) + 1000 + 100 * step
            bank.append(nc, nl, nid, scales=ns)
            for j, i in enumerate(nid.tolist()):
                blocks[i] = (nc[int(no[j]) * kv * hd:int(no[j + 1]) * kv * hd],
                             ns[int(no[j]) * kv:int(no[j + 1]) * kv])
            if step == 1:
                bank.compact()
            order = sorted(blocks)
            cat = np.concatenate([blocks[i][0] for i in order])
            scat = np.concatenate([blocks[i][1] for i in order])
            lens_now = [blocks[i][0].size // (kv * hd) for i in order]
            o = np.zeros(len(order) + 1, np.uint64)
            o[1:] = np.cumsum(lens_now)
            res = bank.route(qs, 5)
            want, wsc, _ = oracle.gqa_route(cat, oracle.I8, o, kv, hd, qs, 5, scales=scat,
                                            scale_dtype="f16", group_size=hd,
                                            node_ids=np.asarray(order, np.uint64))
            assert_same(res, want, wsc)


@pytest.mark.parametrize("route_chunk,cand_chunk", [("512", "64"), ("64", "512"), ("256", "16")])
def test_candidate_items_apart_from_route_items(hip_lib, monkeypatch, route_chunk, cand_chunk):
    # The bound-and-verify exact step cuts its candidates into items of its
    # own length (GRM_HIP_GQA_CAND_CHUNK), sized apart from the route's
    # items (GRM_HIP_GQA_CHUNK): shorter, longer, and the shortest allowed.
    monkeypatch.setenv("GRM_HIP_GQA_BOUND", "1")
    monkeypatch.setenv("GRM_HIP_GQA_CHUNK", route_chunk)
    monkeypatch.setenv("GRM_HIP_GQA_CAND_CHUNK", cand_chunk)
    rng = np.random.default_rng(int(route_chunk) + int(cand_chunk))
    keys, offs = ragged(rng, 120, 8, 128, 1, 700)
    qs = rng.standard_normal((8, 32, 1, 128)).astype(np.float32)  # 32 columns per kv head
    with GqaNodeBank(keys, offs, kv_heads=8, head_dim=128, dtype="bf16") as bank:
        res = bank.route(qs, 6)
        stats = bank.route_stats()
    ids, sc, _ = oracle.gqa_route(oracle.bf16_bits(keys), oracle.BF16, offs, 8, 128, qs, 6)
    assert_same(res, ids, sc)
    assert stats["bound_verify"] > 0
