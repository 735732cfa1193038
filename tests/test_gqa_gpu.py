"""Ragged GQA route parity on the GPU: the HIP library against the fp64 oracle.

Bar: node ids bit-exact (ties to the lowest node id), scores bit-exact (the
kernels evaluate gqa_raw_score, cpp/grm_runtime.cpp:2980-3029, in its
order).  Hand cases come from the reference tests:
tests/test_gqa_ragged_cuda_bank.py:213-229 ([1, 2, 0]) and :441-454 (ties
[0, 1, 2]).
"""

import numpy as np
import pytest

import oracle
from graftrepository_amd import GqaNodeBank, workloads as wl
from graftrepository_amd.gqa_probe import HipProbe
from graftrepository_amd.grm_hip_router import CudaGQARouteSidecar
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


@pytest.mark.parametrize("kv,H,Qt,hd", [(1, 1, 1, 8), (2, 8, 2, 16),
                                        (8, 32, 1, 128), (4, 16, 4, 64),
                                        (8, 8, 3, 32)])
def test_f32_ragged_parity(hip_lib, kv, H, Qt, hd):
    rng = np.random.default_rng(kv * 100 + H + Qt + hd)
    keys, offs = ragged(rng, 150, kv, hd, 0, 150)
    qs = rng.standard_normal((3, H, Qt, hd)).astype(np.float32)
    with GqaNodeBank(keys, offs, kv_heads=kv, head_dim=hd) as bank:
        res = bank.route(qs, 6)
    ids, sc, _ = oracle.gqa_route(keys, oracle.F32, offs, kv, hd, qs, 6)
    assert_same(res, ids, sc)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_half_banks_parity(hip_lib, dtype):
    lens = wl.gqa_lengths(300, seed=7, lo=1, hi=200)
    keys, offs = wl.gqa_bank(lens, 8, 128, seed=7, dtype=dtype)
    qs = wl.gqa_queries(2, 32, 1, 128, seed=7, dtype="bf16")
    with GqaNodeBank(keys, offs, kv_heads=8, head_dim=128, dtype=dtype) as bank:
        res = bank.route(qs, 5, query_dtype="bf16")
    code = oracle.BF16 if dtype == "bf16" else oracle.F16
    ids, sc, _ = oracle.gqa_route(keys, code, offs, 8, 128,
                                  bf16_bits_to_f32(qs).reshape(qs.shape), 5)
    assert_same(res, ids, sc)


@pytest.mark.parametrize("group,scale_dtype", [(32, "f32"), (128, "f16"),
                                               (64, "f32")])
def test_int8_bank_parity(hip_lib, group, scale_dtype):
    rng = np.random.default_rng(group)
    keys, offs = ragged(rng, 200, 8, 128, 1, 120)
    codes, scales = oracle.quantize_int8(keys.reshape(-1, 128), group,
                                         scale_dtype)
    qs = rng.standard_normal((2, 32, 1, 128)).astype(np.float32)
    with GqaNodeBank(codes, offs, kv_heads=8, head_dim=128, dtype="i8",
                     scales=scales, scale_dtype=scale_dtype,
                     group_size=group) as bank:
        res = bank.route(qs, 5)
    sd = "f16" if scale_dtype == "f16" else "f32"
    ids, sc, _ = oracle.gqa_route(codes, oracle.I8, offs, 8, 128, qs, 5,
                                  scales=scales, scale_dtype=sd,
                                  group_size=group)
    assert_same(res, ids, sc)


def test_reference_hand_cases(hip_lib):
    # tests/test_gqa_ragged_cuda_bank.py:213-229
    rows = [np.asarray([[[0.05, 0.0]]], np.float32),
            np.asarray([[[0.1, 0.0], [2.0, 0.0], [0.3, 0.0]]], np.float32),
            np.asarray([[[0.4, 0.0], [0.2, 0.0]]], np.float32)]
    q = np.asarray([[[1.0, 0.0]]], np.float32)
    # head_dim 2 is below the 16-byte row granule; pad with zero dims, which
    # leaves every dot product unchanged.
    pad = lambda a: np.concatenate([a, np.zeros(a.shape[:-1] + (2,), np.float32)], -1)
    keys = np.concatenate([pad(r).reshape(-1) for r in rows])
    offs = np.asarray([0, 1, 4, 6], np.uint64)
    with GqaNodeBank(keys, offs, kv_heads=1, head_dim=4) as bank:
        assert bank.route(pad(q), 3).ids[0].tolist() == [1, 2, 0]
        assert bank.route(pad(q), 2).ids[0].tolist() == [1, 2]
    # :441-454 identical rows tie to the lowest id
    row = pad(np.asarray([[[1.0, 0.0], [0.0, 0.5]]], np.float32))
    keys = np.concatenate([row.reshape(-1)] * 3)
    offs = np.asarray([0, 2, 4, 6], np.uint64)
    with GqaNodeBank(keys, offs, kv_heads=1, head_dim=4) as bank:
        assert bank.route(pad(q), 3).ids[0].tolist() == [0, 1, 2]


def test_empty_nodes_nonfinite_keys_and_query(hip_lib):
    rng = np.random.default_rng(3)
    kv, hd, H = 2, 16, 4
    lens = np.asarray([3, 0, 5, 2, 0, 4], np.uint64)
    offs = np.zeros(lens.size + 1, np.uint64)
    offs[1:] = np.cumsum(lens)
    keys = rng.standard_normal(int(offs[-1]) * kv * hd).astype(np.float32)
    # poison node 3
    keys[int(offs[3]) * kv * hd + 5] = np.nan
    q = rng.standard_normal((1, H, 1, hd)).astype(np.float32)
    with GqaNodeBank(keys, offs, kv_heads=kv, head_dim=hd) as bank:
        res = bank.route(q, 5)
        ids, sc, _ = oracle.gqa_route(keys, oracle.F32, offs, kv, hd, q, 5)
        assert_same(res, ids, sc)
        assert 3 not in res.ids[0].tolist()
        assert {1, 4} <= set(res.ids[0].tolist())  # empty nodes score 0.0
        bad = q.copy()
        bad[0, 1, 0, 2] = np.inf
        res = bank.route(bad, 5)
        ids, sc, _ = oracle.gqa_route(keys, oracle.F32, offs, kv, hd, bad, 5)
        assert_same(res, ids, sc)
        assert sorted(res.ids[0][:2].tolist()) == [1, 4]


def test_dense_reference_surface(hip_lib):
    rng = np.random.default_rng(12)
    bank_np = rng.standard_normal((64, 4, 32, 64)).astype(np.float32)
    bank_np[:, :, 20:, :] = 0.0  # zero-padded tails
    qs = rng.standard_normal((4, 16, 2, 64)).astype(np.float32)
    node_ids = np.arange(64, dtype=np.uint64) * 7
    sidecar = CudaGQARouteSidecar.build()
    bank = sidecar.create_bank(bank_np, node_ids)
    mapped, receipt = bank.route_topk(qs, topk=4, warmup=1)
    offs = np.arange(65, dtype=np.uint64) * 32
    want, _, _ = oracle.gqa_route(bank_np.reshape(-1), oracle.F32, offs, 4, 64,
                                  qs, 4)
    np.testing.assert_array_equal(mapped, node_ids[want])
    assert receipt.measured_queries == 3
    probe = HipProbe()
    dq = probe.upload_queries(qs)
    mapped_d, _ = bank.route_topk_device(dq, topk=4)
    np.testing.assert_array_equal(mapped_d, mapped)
    dq.close()
    bank.close()


def test_append_evict_compact(hip_lib):
    rng = np.random.default_rng(77)
    kv, hd, H = 4, 32, 8
    keys, offs = ragged(rng, 80, kv, hd, 1, 60)
    ids0 = np.arange(80, dtype=np.uint64) + 1
    q = rng.standard_normal((2, H, 1, hd)).astype(np.float32)
    blocks = {int(i): keys[int(offs[j]) * kv * hd:int(offs[j + 1]) * kv * hd]
              for j, i in enumerate(ids0)}
    with GqaNodeBank(keys, offs, kv_heads=kv, head_dim=hd, node_ids=ids0,
                     capacity_nodes=200, capacity_tokens=20000) as bank:
        for step in range(3):
            ev = rng.choice(sorted(blocks), size=10, replace=False)
            bank.evict(ev)
            for i in ev.tolist():
                del blocks[i]
            lens = rng.integers(0, 70, size=12)
            new = [rng.standard_normal(int(L) * kv * hd).astype(np.float32)
                   for L in lens]
            nid = np.arange(12, dtype=np.uint64) + 1000 + 100 * step
            bank.append(np.concatenate(new), lens, nid)
            for i, b in zip(nid.tolist(), new):
                blocks[i] = b
            if step == 1:
                bank.compact()
            order = sorted(blocks)
            cat = np.concatenate([blocks[i] for i in order])
            lens_now = [blocks[i].size // (kv * hd) for i in order]
            o = np.zeros(len(order) + 1, np.uint64)
            o[1:] = np.cumsum(lens_now)
            res = bank.route(q, 7)
            want, wsc, _ = oracle.gqa_route(cat, oracle.F32, o, kv, hd, q, 7,
                                            node_ids=np.asarray(order, np.uint64))
            assert_same(res, want, wsc)
        assert bank.info()["live"] == len(blocks)


@pytest.mark.parametrize("Qt", [1, 4])
def test_ragged_config_parity(hip_lib, Qt):
    cfg = wl.GQA_RAGGED
    kv = cfg["layers"] * cfg["kv_heads"]
    H = cfg["layers"] * cfg["heads"]
    lens = wl.gqa_lengths(cfg["nodes"], cfg["seed"], lo=cfg["lo"], hi=cfg["hi"])
    keys, offs = wl.gqa_bank(lens, kv, cfg["head_dim"], cfg["seed"])
    qs = wl.gqa_queries(2, H, Qt, cfg["head_dim"], cfg["seed"] + Qt - 1)
    with GqaNodeBank(keys, offs, kv_heads=kv, head_dim=cfg["head_dim"],
                     dtype="bf16") as bank:
        res = bank.route(qs, cfg["topk"], query_dtype="bf16")
        one = bank.route(qs[:1], cfg["topk"], query_dtype="bf16", timed=False)
    ids, sc, _ = oracle.gqa_route(keys, oracle.BF16, offs, kv, cfg["head_dim"],
                                  bf16_bits_to_f32(qs).reshape(qs.shape),
                                  cfg["topk"])
    assert_same(res, ids, sc)
    assert_same(one, ids[:1], sc[:1])


@pytest.mark.parametrize("Qt", [1, 4])
def test_screen_path_matches_exact_path(hip_lib, monkeypatch, Qt):
    lens = wl.gqa_lengths(400, seed=31, lo=1, hi=300)
    keys, offs = wl.gqa_bank(lens, 16, 128, seed=31, dtype="bf16")
    qs = wl.gqa_queries(20, 64, Qt, 128, seed=31, dtype="bf16")  # 2 screen batches
    results = {}
    for screen in ("1", "0"):
        monkeypatch.setenv("GRM_HIP_GQA_SCREEN", screen)
        with GqaNodeBank(keys, offs, kv_heads=16, head_dim=128,
                         dtype="bf16") as bank:
            results[screen] = bank.route(qs, 5, query_dtype="bf16", warmup=3)
    ids, sc, _ = oracle.gqa_route(keys, oracle.BF16, offs, 16, 128,
                                  bf16_bits_to_f32(qs).reshape(qs.shape), 5)
    for r in results.values():
        assert_same(r, ids, sc)


def test_tied_nodes_order_by_lowest_id(hip_lib):
    # 100 identical nodes tie exactly on the screen-and-refine path; the
    # exact maxima are equal, so the order falls to the node ids.
    rng = np.random.default_rng(8)
    block = rng.standard_normal(8 * 40 * 64).astype(np.float32)
    others = rng.standard_normal(8 * 40 * 64 * 5).astype(np.float32) * 0.1
    keys = np.concatenate([np.tile(block, 100), others])
    offs = np.arange(106, dtype=np.uint64) * 40
    ids = (np.arange(105, dtype=np.uint64)[::-1] + 7).copy()
    q = rng.standard_normal((1, 16, 1, 64)).astype(np.float32)
    with GqaNodeBank(keys, offs, kv_heads=8, head_dim=64, dtype="bf16",
                     node_ids=ids) as bank:
        res = bank.route(q, 10)
    want, wsc, _ = oracle.gqa_route(oracle.bf16_bits(keys), oracle.BF16, offs,
                                    8, 64, q, 10, node_ids=ids)
    assert_same(res, want, wsc)
    assert res.ids[0].tolist() == sorted(ids[:100].tolist())[:10]


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_f32_queries_on_half_banks(hip_lib, dtype):
    # fp32 query values are converted for the matrix cores; the bound covers
    # the conversion and the exact rescore uses the fp32 values.
    lens = wl.gqa_lengths(200, seed=41, lo=8, hi=128)
    keys, offs = wl.gqa_bank(lens, 8, 64, seed=41, dtype=dtype)
    qs = wl.gqa_queries(3, 32, 2, 64, seed=41, dtype="f32")
    with GqaNodeBank(keys, offs, kv_heads=8, head_dim=64, dtype=dtype) as bank:
        res = bank.route(qs, 4)
    code = oracle.BF16 if dtype == "bf16" else oracle.F16
    ids, sc, _ = oracle.gqa_route(keys, code, offs, 8, 64, qs, 4)
    assert_same(res, ids, sc)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_repeated_tokens_within_nodes(hip_lib, dtype):
    # Nodes whose key tokens repeat: screened values tie three or more ways,
    # so the item is screened again and every candidate is recomputed.
    rng = np.random.default_rng(17)
    kv, hd, H = 4, 64, 16
    lens = rng.integers(1, 300, size=60).astype(np.uint64)
    lens[:4] = [1, 16, 17, 299]
    offs = np.zeros(lens.size + 1, np.uint64)
    offs[1:] = np.cumsum(lens)
    blocks = []
    for i, L in enumerate(lens.tolist()):
        if i % 3 == 0:  # one token repeated L times per kv head
            tok = rng.standard_normal((kv, 1, hd)).astype(np.float32)
            blocks.append(np.repeat(tok, L, axis=1))
        elif i % 3 == 1:  # a few distinct tokens, each repeated
            toks = rng.standard_normal((kv, 3, hd)).astype(np.float32)
            blocks.append(toks[:, rng.integers(0, 3, size=L), :])
        else:
            blocks.append(rng.standard_normal((kv, L, hd)).astype(np.float32))
    keys = np.concatenate([b.reshape(-1) for b in blocks])
    bits = oracle.bf16_bits(keys) if dtype == "bf16" else oracle.f16_bits(keys)
    code = oracle.BF16 if dtype == "bf16" else oracle.F16
    qs = rng.standard_normal((3, H, 2, hd)).astype(np.float32)
    with GqaNodeBank(bits, offs, kv_heads=kv, head_dim=hd, dtype=dtype) as bank:
        res = bank.route(qs, 8)
    ids, sc, _ = oracle.gqa_route(bits, code, offs, kv, hd, qs, 8)
    assert_same(res, ids, sc)


@pytest.mark.parametrize("scale", [3.0e6, 1.0e-7])
def test_f16_bank_queries_outside_half_range(hip_lib, scale):
    # Query values beyond (or far below) the fp16 range are screened with a
    # power-of-two column scale; the result still follows the fp64 law.
    lens = wl.gqa_lengths(120, seed=51, lo=1, hi=100)
    keys, offs = wl.gqa_bank(lens, 4, 128, seed=51, dtype="f16")
    qs = wl.gqa_queries(2, 16, 1, 128, seed=51, dtype="f32") * np.float32(scale)
    qs[0, 3, 0, 7] = np.float32(70000.0 * max(scale, 1.0))
    with GqaNodeBank(keys, offs, kv_heads=4, head_dim=128, dtype="f16") as bank:
        res = bank.route(qs, 6)
    ids, sc, _ = oracle.gqa_route(keys, oracle.F16, offs, 4, 128, qs, 6)
    assert_same(res, ids, sc)


def test_int8_bank_batched_queries(hip_lib):
    # 16 queries x 4 heads per kv head = 64 query columns in one pass.
    rng = np.random.default_rng(61)
    keys, offs = ragged(rng, 300, 8, 128, 1, 400)
    codes, scales = oracle.quantize_int8(keys.reshape(-1, 128), 32, "f16")
    qs = rng.standard_normal((16, 32, 1, 128)).astype(np.float32)
    with GqaNodeBank(codes, offs, kv_heads=8, head_dim=128, dtype="i8",
                     scales=scales, scale_dtype="f16", group_size=32) as bank:
        res = bank.route(qs, 5)
    ids, sc, _ = oracle.gqa_route(codes, oracle.I8, offs, 8, 128, qs, 5,
                                  scales=scales, scale_dtype="f16",
                                  group_size=32)
    assert_same(res, ids, sc)


def test_repeated_routes_follow_query_and_bank_changes(hip_lib):
    # Repeated single-query routes on one device buffer read the query and
    # the bank as they are at each call; batched routes run in between.
    # The buffer comes from the library's own upload entry point and is
    # rewritten with hipMemcpy of the runtime the library runs on.
    import ctypes
    from graftrepository_amd.gqa_probe import HipProbe
    lens = wl.gqa_lengths(200, seed=71, lo=1, hi=300)
    keys, offs = wl.gqa_bank(lens, 8, 128, seed=71, dtype="bf16")
    node_ids = np.arange(200, dtype=np.uint64) + 5
    qs = [wl.gqa_queries(1, 32, 1, 128, seed=71 + i, dtype="f32") for i in range(2)]
    hip = ctypes.CDLL("libamdhip64.so.7")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    dq = HipProbe().upload_queries(qs[0])

    def want(q, live):
        blocks = [keys[int(offs[j]) * 8 * 128:int(offs[j + 1]) * 8 * 128] for j in live]
        o = np.zeros(len(live) + 1, np.uint64)
        o[1:] = np.cumsum([lens[j] for j in live])
        return oracle.gqa_route(np.concatenate(blocks), oracle.BF16, o, 8, 128, q, 4,
                                node_ids=node_ids[live])

    live = list(range(200))
    with GqaNodeBank(keys, offs, kv_heads=8, head_dim=128, dtype="bf16",
                     node_ids=node_ids) as bank:
        ids, sc, _ = want(qs[0], live)
        for _ in range(3):
            assert_same(bank.route(dq, 4, on_device=True), ids, sc)
            eager = bank.route(np.concatenate([qs[0], qs[0]]), 4, warmup=1)
            assert_same(eager, np.concatenate([ids, ids]), np.concatenate([sc, sc]))
        assert hip.hipMemcpy(dq.handle, qs[1].ctypes.data, qs[1].nbytes, 1) == 0
        ids, sc, _ = want(qs[1], live)
        assert_same(bank.route(dq, 4, on_device=True), ids, sc)
        bank.evict(node_ids[:7])
        live = live[7:]
        ids, sc, _ = want(qs[1], live)
        for _ in range(2):
            assert_same(bank.route(dq, 4, on_device=True), ids, sc)


@pytest.mark.parametrize("bound", [None, "0"])
def test_untimed_routes_wait_on_completion_flags(hip_lib, monkeypatch, bound):
    # Routes that ask for no device time wait on the finalize blocks'
    # completion flags instead of a stream event: the same results as timed
    # routes, for one query, several, several screen passes (bound "0"
    # keeps every batch on the screen-and-refine path, 16 queries a pass)
    # and batches that take the bound-and-verify path, across bank changes.
    if bound is not None:
        monkeypatch.setenv("GRM_HIP_GQA_BOUND", bound)
    lens = wl.gqa_lengths(300, seed=83, lo=1, hi=400)
    keys, offs = wl.gqa_bank(lens, 8, 128, seed=83, dtype="bf16")
    node_ids = np.arange(300, dtype=np.uint64) * 3 + 1
    qs = wl.gqa_queries(20, 32, 1, 128, seed=83, dtype="bf16")
    qf = bf16_bits_to_f32(qs).reshape(qs.shape)

    def want(q, live):
        blocks = [keys[int(offs[j]) * 8 * 128:int(offs[j + 1]) * 8 * 128] for j in live]
        o = np.zeros(len(live) + 1, np.uint64)
        o[1:] = np.cumsum([lens[j] for j in live])
        return oracle.gqa_route(np.concatenate(blocks), oracle.BF16, o, 8, 128, q, 5,
                                node_ids=node_ids[live])

    live = list(range(300))
    with GqaNodeBank(keys, offs, kv_heads=8, head_dim=128, dtype="bf16",
                     node_ids=node_ids) as bank:
        for step in range(2):
            for n, warm in ((1, 0), (3, 0), (2, 1), (6, 0), (20, 2)):
                ids, sc, _ = want(qf[:n], live)
                for timed in (False, True, False):
                    r = bank.route(qs[:n], 5, query_dtype="bf16", warmup=warm, timed=timed)
                    assert_same(r, ids, sc)
                    assert np.isnan(r.device_ms) != timed
            if step == 0:
                bank.evict(node_ids[10:40])
                live = live[:10] + live[40:]


@pytest.mark.parametrize("path", ["screen", "exact"])
@pytest.mark.parametrize("chunk", [None, "256"])
@pytest.mark.parametrize("Qt", [1, 4])
def test_long_nodes_span_several_work_items(hip_lib, monkeypatch, Qt, chunk, path):
    # Screen and refine, and the exact fp64 path, over nodes longer than one
    # work item (512 tokens by default for bf16 banks, 256 when set): each
    # item yields its own per-(node, head) maxima, which combine across the
    # node's items.
    monkeypatch.setenv("GRM_HIP_GQA_SCREEN", "1" if path == "screen" else "0")
    monkeypatch.setenv("GRM_HIP_GQA_BOUND", "0")
    if chunk is None:
        monkeypatch.delenv("GRM_HIP_GQA_CHUNK", raising=False)
    else:
        monkeypatch.setenv("GRM_HIP_GQA_CHUNK", chunk)
    rng = np.random.default_rng(900 + Qt)
    kv, hd, H = 4, 128, 16
    keys, offs = ragged(rng, 60, kv, hd, 1, 1500)
    lens = np.diff(offs)
    # the best token of some nodes sits in a late item
    for i in range(0, 60, 7):
        if lens[i] > 1100:
            blk = keys[int(offs[i]) * kv * hd:int(offs[i + 1]) * kv * hd].reshape(kv, int(lens[i]), hd)
            blk[:, 1050] *= 3.0
    qs = rng.standard_normal((2, H, Qt, hd)).astype(np.float32)
    with GqaNodeBank(keys, offs, kv_heads=kv, head_dim=hd, dtype="bf16") as bank:
        res = bank.route(qs, 7)
        one = bank.route(qs[:1], 7, timed=False)
        stats = bank.route_stats()
    ids, sc, _ = oracle.gqa_route(oracle.bf16_bits(keys), oracle.BF16, offs, kv, hd, qs, 7)
    assert_same(res, ids, sc)
    assert_same(one, ids[:1], sc[:1])
    if path == "screen":
        assert stats["screen_refine"] > 0 and stats["exact"] == 0
    else:
        assert stats["exact"] > 0 and stats["screen_refine"] == 0
