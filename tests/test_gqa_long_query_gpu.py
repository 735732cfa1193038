"""GQA routes whose query spans many tokens, on the GPU against the oracle.

The reference's probe key is the layer-0 query over the whole prompt,
[H, L, hd] (core/graft_arena.py:2876-2879, core/kv_graft.py:146-171), and
its sidecar takes any query_tokens (scripts/grm_gqa_cuda_probe.py:376-400).
The library routes a query wider than one pass (64 query columns per kv
head on the screen paths -- 128 on a single query's screen-only passes at
head dims up to 128 -- and 32 on the exact path) in passes over runs of its
tokens -- or of its heads, when one token's R heads are already too many --
folded into the same per-(node, head) maxima.  Bar: ids and score bits
equal to the oracle's fp64 law (cpp/grm_runtime.cpp:2980-3029).
"""

import numpy as np
import pytest

import oracle
from graftrepository_amd import GqaNodeBank, workloads as wl
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


def c4_bank(nodes, hi, seed):
    """The 512-node workload's geometry (4 routing layers x 8 kv heads x
    128, 32 query heads per layer: R = 4) on fewer nodes."""
    cfg = wl.GQA_RAGGED
    kv = cfg["layers"] * cfg["kv_heads"]
    H = cfg["layers"] * cfg["heads"]
    lens = wl.gqa_lengths(nodes, seed, lo=cfg["lo"], hi=hi)
    keys, offs = wl.gqa_bank(lens, kv, cfg["head_dim"], seed)
    return keys, offs, kv, H, cfg["head_dim"]


@pytest.fixture(params=["screen", "screen-all-columns", "refine", "exact"])
def path(request, monkeypatch):
    # screen: the default choice (bound and verify for these widths: its
    # screen in passes of 128 columns, or 4 passes of 64 to a launch, then
    # the law on the columns of each candidate that the screen cannot rule
    # out); screen-all-columns: the screen in passes of 64, two to a
    # launch, the law on every column in passes of 32;
    # refine: screen and refine in passes; exact: the fp64 kernel
    narrow = request.param == "screen-all-columns"
    monkeypatch.setenv("GRM_HIP_GQA_SCREEN", "0" if request.param == "exact" else "1")
    monkeypatch.setenv("GRM_HIP_GQA_SPARSE", "0" if narrow else "1")
    monkeypatch.setenv("GRM_HIP_GQA_WIDE_SMAX", "0" if narrow else "1")
    # narrow: split launches of 2 passes; otherwise the default (4 passes
    # of 64 columns to a launch from 4 passes on, else passes of 128)
    monkeypatch.setenv("GRM_HIP_GQA_SMAX_SPLIT", "2" if narrow else "4")
    if request.param == "refine":
        monkeypatch.setenv("GRM_HIP_GQA_BOUND", "0")
    else:
        monkeypatch.delenv("GRM_HIP_GQA_BOUND", raising=False)
    return request.param


@pytest.mark.parametrize("Qt,nodes,hi", [(9, 96, 512), (33, 96, 512), (64, 64, 512),
                                         (256, 24, 256)])
def test_c4_geometry_long_queries(hip_lib, path, Qt, nodes, hi):
    keys, offs, kv, H, hd = c4_bank(nodes, hi, seed=40 + Qt)
    qs = wl.gqa_queries(1, H, Qt, hd, seed=50 + Qt)
    with GqaNodeBank(keys, offs, kv_heads=kv, head_dim=hd, dtype="bf16") as bank:
        res = bank.route(qs, 3, query_dtype="bf16")
        untimed = bank.route(qs, 3, query_dtype="bf16", timed=False)
    ids, sc, _ = oracle.gqa_route(keys, oracle.BF16, offs, kv, hd,
                                  bf16_bits_to_f32(qs).reshape(qs.shape), 3)
    assert_same(res, ids, sc)
    assert_same(untimed, ids, sc)


def test_head_dim_256_sixteen_heads(hip_lib, path):
    # 16 query heads on 4 kv heads (R = 4), head_dim 256, 24 query tokens:
    # 96 columns per kv head, two screen passes or three exact ones
    lens = wl.gqa_lengths(120, seed=61, lo=1, hi=300)
    keys, offs = wl.gqa_bank(lens, 4, 256, seed=61, dtype="bf16")
    qs = wl.gqa_queries(2, 16, 24, 256, seed=61, dtype="bf16")
    with GqaNodeBank(keys, offs, kv_heads=4, head_dim=256, dtype="bf16") as bank:
        res = bank.route(qs, 5, query_dtype="bf16")
    ids, sc, _ = oracle.gqa_route(keys, oracle.BF16, offs, 4, 256,
                                  bf16_bits_to_f32(qs).reshape(qs.shape), 5)
    assert_same(res, ids, sc)


@pytest.mark.parametrize("H,kv,Qt", [(64, 1, 3), (128, 2, 2), (40, 1, 5)])
def test_more_heads_per_kv_head_than_one_pass(hip_lib, path, H, kv, Qt):
    # R = 64, 64 and 40: the exact path splits each token's heads into
    # passes of 32, the screen path takes one token per pass
    rng = np.random.default_rng(H + kv + Qt)
    lens = rng.integers(0, 90, size=80).astype(np.uint64)
    offs = np.zeros(lens.size + 1, np.uint64)
    offs[1:] = np.cumsum(lens)
    keys = wl.gqa_bank(lens, kv, 64, seed=H + Qt, dtype="bf16")[0]
    qs = wl.gqa_queries(2, H, Qt, 64, seed=H + Qt, dtype="bf16")
    with GqaNodeBank(keys, offs, kv_heads=kv, head_dim=64, dtype="bf16") as bank:
        res = bank.route(qs, 4, query_dtype="bf16")
    ids, sc, _ = oracle.gqa_route(keys, oracle.BF16, offs, kv, 64,
                                  bf16_bits_to_f32(qs).reshape(qs.shape), 4)
    assert_same(res, ids, sc)


def test_f32_bank_long_query(hip_lib):
    rng = np.random.default_rng(71)
    lens = rng.integers(1, 200, size=100).astype(np.uint64)
    offs = np.zeros(lens.size + 1, np.uint64)
    offs[1:] = np.cumsum(lens)
    keys = rng.standard_normal(int(offs[-1]) * 8 * 128).astype(np.float32)
    qs = rng.standard_normal((2, 32, 20, 128)).astype(np.float32)
    with GqaNodeBank(keys, offs, kv_heads=8, head_dim=128) as bank:
        res = bank.route(qs, 6)
    ids, sc, _ = oracle.gqa_route(keys, oracle.F32, offs, 8, 128, qs, 6)
    assert_same(res, ids, sc)


@pytest.mark.parametrize("bound", ["1", "auto"])
def test_int8_bank_batched_long_queries(hip_lib, monkeypatch, bound):
    # 20 tokens x R = 4: 80 columns per query; queries that do not fit one
    # screen pass are routed one by one (through bound and verify, its
    # screen in one pass of 80 columns and its exact pass in passes of 32)
    if bound == "auto":
        monkeypatch.delenv("GRM_HIP_GQA_BOUND", raising=False)
    else:
        monkeypatch.setenv("GRM_HIP_GQA_BOUND", bound)
    rng = np.random.default_rng(81)
    lens = rng.integers(1, 150, size=150).astype(np.uint64)
    offs = np.zeros(lens.size + 1, np.uint64)
    offs[1:] = np.cumsum(lens)
    vals = rng.standard_normal((int(offs[-1]) * 8, 128)).astype(np.float32)
    codes, scales = oracle.quantize_int8(vals, 128, "f16")
    qs = wl.gqa_queries(3, 32, 20, 128, seed=81, dtype="bf16")
    with GqaNodeBank(codes, offs, kv_heads=8, head_dim=128, dtype="i8", scales=scales,
                     scale_dtype="f16", group_size=128) as bank:
        res = bank.route(qs, 5, query_dtype="bf16", warmup=1)
    ids, sc, _ = oracle.gqa_route(codes, oracle.I8, offs, 8, 128,
                                  bf16_bits_to_f32(qs).reshape(qs.shape), 5,
                                  scales=scales, scale_dtype="f16", group_size=128)
    assert_same(res, ids, sc)


def test_non_finite_value_in_a_late_pass(hip_lib, path):
    # a NaN in the last token of one head lies in the last pass only; the
    # query flag it raises must survive the passes, so nothing is ranked
    lens = wl.gqa_lengths(40, seed=91, lo=1, hi=100)
    keys, offs = wl.gqa_bank(lens, 8, 128, seed=91, dtype="bf16")
    qf = bf16_bits_to_f32(wl.gqa_queries(2, 32, 40, 128, seed=91)).reshape(2, 32, 40, 128)
    qf[1, 29, 39, 5] = np.nan
    with GqaNodeBank(keys, offs, kv_heads=8, head_dim=128, dtype="bf16") as bank:
        res = bank.route(qf, 3)
    ids, sc, _ = oracle.gqa_route(keys, oracle.BF16, offs, 8, 128, qf, 3)
    assert_same(res, ids, sc)
    assert np.all(res.ids[1] == NO_ID) and np.all(res.ids[0] != NO_ID)


def test_reference_surface_prompt_length_query(hip_lib):
    # the reference's dense f32 bank (zero-padded to the longest node) and
    # a 40-token query through the sidecar surface: row indices
    rng = np.random.default_rng(101)
    n, kv, T, hd = 64, 8, 96, 64
    dense = np.zeros((n, kv, T, hd), np.float32)
    lens = rng.integers(1, T + 1, size=n)
    for i, L in enumerate(lens):
        dense[i, :, :L] = rng.standard_normal((kv, L, hd))
    qs = rng.standard_normal((2, 32, 40, hd)).astype(np.float32)
    sidecar = CudaGQARouteSidecar.build()
    bank = sidecar.create_bank(dense, np.arange(n, dtype=np.uint64) + 7)
    mapped, _ = bank.route_topk(qs, topk=4)
    offs = np.arange(n + 1, dtype=np.uint64) * T
    want, _, _ = oracle.gqa_route(dense.reshape(-1), oracle.F32, offs, kv, hd, qs, 4)
    np.testing.assert_array_equal(mapped, want + 7)
    bank.close()


def test_query_wider_than_the_staged_rows(hip_lib, path):
    # 4 heads per kv head x 1024 query tokens: 4096 columns per kv head,
    # past the query-row staging of the exact step's double rows (they go
    # straight to device memory), and 64 screen passes
    lens = wl.gqa_lengths(24, seed=91, lo=1, hi=40)
    keys, offs = wl.gqa_bank(lens, 4, 64, seed=91, dtype="bf16")
    qs = wl.gqa_queries(1, 16, 1024, 64, seed=92, dtype="bf16")
    with GqaNodeBank(keys, offs, kv_heads=4, head_dim=64, dtype="bf16") as bank:
        res = bank.route(qs, 3, query_dtype="bf16")
    ids, sc, _ = oracle.gqa_route(keys, oracle.BF16, offs, 4, 64,
                                  bf16_bits_to_f32(qs).reshape(qs.shape), 3)
    assert_same(res, ids, sc)
