"""Pin the CPU oracle before trusting it (CPU only).

* reference goldens: route orders produced by the reference's own C++
  router (tests/golden/route_goldens.json, written by make_golden.py from
  cpp/grm_runtime.cpp built into oracle/_ref);
* the reference router itself when oracle/_ref is built here: randomized
  cross-checks of ids;
* closed forms the mathematics fixes (orthonormal rows, Pythagorean norms,
  single-token GQA), chosen so a dropped norm, a wrong sign, a missing
  abs or a transposed head mapping fails;
* the storage laws: fp16 conversion against numpy, bf16 rounding against
  torch, the INT8 quantiser's round-trip invariants
  (tests/test_graft_quant_format.py:54-78 in the reference).
"""

import json
from pathlib import Path

import numpy as np
import pytest

import oracle
from graftrepository_amd.workloads import digest
from tests.golden.cases import (GQA_CASES, MLA_CASES, gqa_inputs, gqa_storage,
                                mla_inputs)

GOLDEN = json.loads((Path(__file__).parent / "golden" / "route_goldens.json")
                    .read_text())
NO_ID = np.iinfo(np.uint64).max


def _case(kind, name):
    return next(c for c in GOLDEN[kind] if c["name"] == name)


@pytest.mark.parametrize("case", MLA_CASES, ids=[c["name"] for c in MLA_CASES])
def test_mla_oracle_matches_reference_goldens(case):
    rows, qs = mla_inputs(case)
    gold = _case("mla", case["name"])
    assert digest(rows, qs) == gold["digest"], "input generator drifted"
    ids, _, counts = oracle.mla_route(rows, qs, case["topk"])
    for qi, want in enumerate(gold["ids"]):
        got = [int(x) for x in ids[qi][:counts[qi]]]
        assert got == want


@pytest.mark.parametrize("case", GQA_CASES, ids=[c["name"] for c in GQA_CASES])
def test_gqa_oracle_matches_reference_goldens(case):
    blocks, qs = gqa_inputs(case)
    gold = _case("gqa", case["name"])
    flat = np.concatenate([b.reshape(-1) for b in blocks])
    assert digest(flat, qs) == gold["digest"], "input generator drifted"
    keys, offs, scales, code, _ = gqa_storage(case)
    ids, _, counts = oracle.gqa_route(
        keys, code, offs, case["kv"], case["hd"], qs, case["topk"],
        scales=scales, scale_dtype=case.get("scale_dtype", "f32"),
        group_size=case.get("group", 0))
    for qi, want in enumerate(gold["ids_fp64_law"]):
        assert [int(x) for x in ids[qi][:counts[qi]]] == want
    # The reference's fp32 arena path agrees on these inputs (no near ties).
    assert gold["ids_fp32_arena"] == gold["ids_fp64_law"]


def _ref_or_skip():
    import oracle.ref as ref
    if not oracle.REF_LIB_PATH.exists():
        pytest.skip("reference CPU router not built (oracle/_ref)")
    return ref


def test_mla_oracle_matches_reference_router_randomized():
    ref = _ref_or_skip()
    rng = np.random.default_rng(77)
    for trial in range(6):
        n, d = int(rng.integers(1, 400)), int(rng.integers(1, 300))
        rows = rng.standard_normal((n, d)).astype(np.float32)
        if trial % 2:
            rows[rng.integers(0, n, 3)] = rows[0]   # exact duplicates
        q = rng.standard_normal(d).astype(np.float32)
        k = int(min(n, rng.integers(1, 17)))
        ids, _, c = oracle.mla_route(rows, q, k)
        assert [int(x) for x in ids[0][:c[0]]] == ref.mla_route(rows, q, k)


def test_gqa_oracle_matches_reference_router_randomized():
    ref = _ref_or_skip()
    rng = np.random.default_rng(78)
    for _ in range(6):
        kv = int(rng.choice([1, 2, 4]))
        H = kv * int(rng.choice([1, 2, 4]))
        hd, Qt, n = int(rng.choice([4, 8, 16])), int(rng.integers(1, 4)), 30
        lens = rng.integers(1, 20, n)
        blocks = [rng.standard_normal((kv, int(L), hd)).astype(np.float32)
                  for L in lens]
        q = rng.standard_normal((H, Qt, hd)).astype(np.float32)
        offs = np.zeros(n + 1, np.uint64)
        offs[1:] = np.cumsum(lens)
        flat = np.concatenate([b.reshape(-1) for b in blocks])
        ids, _, c = oracle.gqa_route(flat, oracle.F32, offs, kv, hd, q, 9)
        assert [int(x) for x in ids[0][:c[0]]] == ref.gqa_route(
            blocks, q, kv, 9, fp64_gqa=True)


# ------------------------------------------------------------- closed forms

def test_mla_closed_form_orthonormal_and_norms():
    rows = np.zeros((4, 3), np.float32)
    rows[0] = [3, 4, 0]       # norm 5
    rows[1] = [0, 0, 2]       # norm 2
    rows[2] = [-3, -4, 0]     # opposite of row 0
    rows[3] = [0, 5, 12]      # norm 13
    assert oracle.mla_row_norms(rows).tolist() == [5.0, 2.0, 5.0, 13.0]
    q = np.asarray([3, 4, 0], np.float32)
    s = oracle.mla_scores(rows, q)[0]
    qn = 5.0
    want = [25.0 / (qn * 5.0 + 1e-8), 0.0, -25.0 / (qn * 5.0 + 1e-8),
            20.0 / (qn * 13.0 + 1e-8)]
    np.testing.assert_array_equal(s, np.asarray(want, np.float32))
    ids, sc, _ = oracle.mla_route(rows, q, 4)
    assert ids[0].tolist() == [0, 3, 1, 2]


def test_gqa_closed_form_single_token():
    # One key token per node: best_h = |q_h . k_{h/R}| / sqrt(hd).
    rng = np.random.default_rng(5)
    kv, R, hd = 2, 3, 8
    H = kv * R
    q = rng.standard_normal((H, 1, hd)).astype(np.float32)
    k = rng.standard_normal((kv, 1, hd)).astype(np.float32)
    want = np.mean([abs(float(np.dot(q[h, 0].astype(np.float64),
                                     k[h // R, 0].astype(np.float64))))
                    / np.sqrt(hd) for h in range(H)])
    offs = np.asarray([0, 1], np.uint64)
    got = oracle.gqa_scores(k.reshape(-1), oracle.F32, offs, kv, hd, q)[0, 0]
    assert abs(float(got) - want) <= 1e-6 * abs(want)
    # sign flip of the key leaves the score unchanged (|q.k|)
    got_neg = oracle.gqa_scores((-k).reshape(-1), oracle.F32, offs, kv, hd, q)
    assert got_neg[0, 0] == got


def test_gqa_empty_and_nonfinite_nodes():
    kv, hd, H = 1, 4, 1
    q = np.ones((1, 1, hd), np.float32)
    keys = np.asarray([1, 0, 0, 0, np.nan, 0, 0, 0], np.float32)
    offs = np.asarray([0, 1, 1, 2], np.uint64)   # node 1 has no tokens
    s = oracle.gqa_scores(keys, oracle.F32, offs, kv, hd, q)[0]
    assert s[0] == np.float32(1.0 / 2.0) and s[1] == 0.0 and np.isnan(s[2])


def test_tie_law_and_unfilled_slots():
    scores = np.asarray([0.5, 0.7, 0.7, np.nan, 0.7, -np.inf], np.float32)
    ids = np.asarray([10, 30, 20, 5, 40, 1], np.uint64)
    out, sc, n = oracle.select_topk(scores, 8, node_ids=ids)
    assert n == 4
    assert out.tolist()[:4] == [20, 30, 40, 10]
    assert all(x == NO_ID for x in out.tolist()[4:])
    assert np.all(np.isnan(sc[4:]))


# ------------------------------------------------------------ storage laws

def test_f16_conversion_matches_numpy():
    # every fp16 bit pattern round-trips (NaN payloads aside)
    allh = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    f = oracle.f16_to_f32(allh)
    np.testing.assert_array_equal(f[~np.isnan(f)],
                                  allh.view(np.float16).astype(np.float32)[~np.isnan(f)])
    finite = ~np.isnan(f)
    np.testing.assert_array_equal(oracle.f16_bits(f[finite]), allh[finite])
    # rounding of fp32 values, including subnormal, tie and overflow edges
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(200_000).astype(np.float32) * 1000,
        rng.standard_normal(200_000).astype(np.float32) * 1e-5,
        np.asarray([65504, 65519.99, 65520, 1e6, 2.0 ** -25, 2.0 ** -24,
                    1.5 * 2.0 ** -24, 2.0 ** -26, -0.0, np.inf, -np.inf],
                   np.float32)])
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(oracle.f16_bits(x), want)


def test_bf16_rounding_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(1)
    x = rng.standard_normal(100_000).astype(np.float32)
    x[:4] = [1.00390625, 1.01171875, -3.0e38, 1e-40]   # ties and extremes
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy()
    np.testing.assert_array_equal(oracle.bf16_bits(x), want.view(np.uint16))


@pytest.mark.parametrize("group,sd", [(32, "f32"), (128, "f16"), (64, "f32")])
def test_int8_quantiser_round_trip_invariants(group, sd):
    rng = np.random.default_rng(group)
    x = rng.standard_normal((257, 128)).astype(np.float32) * 3
    x[7] = 0.0                                            # all-zero group
    codes, scales = oracle.quantize_int8(x, group, sd)
    assert codes.dtype == np.int8 and codes.shape == x.shape
    s = oracle.f16_to_f32(scales) if sd == "f16" else scales
    assert np.all(s[7] == 1.0)
    deq = oracle.dequantize_int8(codes, scales, group, sd)
    err = np.abs(deq - x).reshape(257, -1, group)
    bound = (s.reshape(257, -1, 1) * 0.5 + np.abs(x).reshape(257, -1, group)
             * 2.0 ** -10)
    assert np.all(err <= bound * 1.0001 + 1e-7)
    codes2, scales2 = oracle.quantize_int8(x, group, sd)
    np.testing.assert_array_equal(codes, codes2)
    np.testing.assert_array_equal(scales, scales2)


def test_dequant_law_is_fp16_of_fp32_product():
    codes = np.asarray([[127, -128, 1, -1] * 8], np.int8)
    scales = np.asarray([[0.1]], np.float32)
    got = oracle.dequantize_int8(codes, scales, 32, "f32")
    want = (codes.astype(np.float32) * np.float32(0.1)).astype(np.float16)
    np.testing.assert_array_equal(got, want.astype(np.float32))
