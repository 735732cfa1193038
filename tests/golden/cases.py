"""Golden route cases: parameters and the seeded input generators.

Each case's inputs are regenerated from its parameters; the fixture file
(route_goldens.json) records the sha256 digest of the generated inputs so a
drift in a generator fails loudly instead of comparing different data.
"""

from __future__ import annotations

import numpy as np

import oracle
from graftrepository_amd import workloads as wl

MLA_CASES = [
    dict(name="mla_unit_gauss_288", kind="unit_gauss", nodes=2000, dim=288,
         queries=6, topk=16, seed=101),
    dict(name="mla_small_config", kind="unit_gauss", nodes=10_000, dim=288,
         queries=4, topk=3, seed=1),
    dict(name="mla_raw_gauss_128", kind="raw_gauss", nodes=3000, dim=128,
         queries=4, topk=5, seed=102),
    dict(name="mla_tie_blocks", kind="ties", nodes=1000, dim=64, queries=3,
         topk=16, seed=103),
    dict(name="mla_nan_rows", kind="nan", nodes=500, dim=32, queries=3,
         topk=10, seed=104),
    dict(name="mla_bf16_288", kind="bf16", nodes=2000, dim=288, queries=4,
         topk=8, seed=105),
]

GQA_CASES = [
    dict(name="gqa_small_f32", dtype="f32", nodes=60, kv=2, hd=16, H=8, Qt=2,
         lo=1, hi=40, queries=3, topk=7, seed=201),
    dict(name="gqa_qwen_bf16", dtype="bf16", nodes=40, kv=8, hd=128, H=32,
         Qt=1, lo=16, hi=96, queries=2, topk=5, seed=202),
    dict(name="gqa_stacked_layers_bf16", dtype="bf16", nodes=24, kv=32,
         hd=128, H=128, Qt=1, lo=16, hi=64, queries=2, topk=3, seed=203),
    dict(name="gqa_qt4_f32", dtype="f32", nodes=50, kv=4, hd=32, H=16, Qt=4,
         lo=1, hi=30, queries=2, topk=6, seed=204),
    dict(name="gqa_int8_g32", dtype="i8", nodes=40, kv=8, hd=128, H=32, Qt=1,
         lo=1, hi=50, queries=2, topk=5, seed=205, group=32, scale_dtype="f32"),
    dict(name="gqa_int8_row_f16", dtype="i8", nodes=40, kv=8, hd=128, H=32,
         Qt=1, lo=1, hi=50, queries=2, topk=5, seed=206, group=128,
         scale_dtype="f16"),
]


def mla_inputs(case: dict) -> tuple[np.ndarray, np.ndarray]:
    """Rows [N, D] and queries [Q, D] as float32 values."""
    n, d, q, seed = case["nodes"], case["dim"], case["queries"], case["seed"]
    kind = case["kind"]
    if kind == "unit_gauss":
        return wl.mla_rows(n, d, seed), wl.mla_queries(q, d, seed)
    if kind == "bf16":
        rows = oracle.round_bf16(wl.mla_rows(n, d, seed))
        return rows, oracle.round_bf16(wl.mla_queries(q, d, seed))
    rng = np.random.default_rng(seed)
    if kind == "raw_gauss":
        rows = rng.standard_normal((n, d)).astype(np.float32) * np.float32(3.0)
        return rows, rng.standard_normal((q, d)).astype(np.float32)
    if kind == "ties":
        base = rng.standard_normal((n // 20, d)).astype(np.float32)
        rows = np.ascontiguousarray(np.repeat(base, 20, axis=0))
        qs = base[:q] + np.float32(0.5) * base[q:2 * q]
        return rows, np.ascontiguousarray(qs)
    if kind == "nan":
        rows = rng.standard_normal((n, d)).astype(np.float32)
        rows[::37, 1] = np.nan
        rows[5::41, 0] = np.inf
        return rows, rng.standard_normal((q, d)).astype(np.float32)
    raise ValueError(kind)


def gqa_storage(case: dict):
    """Storage-form bank for the HIP library / oracle: (keys, tok_offsets,
    scales or None, oracle key dtype code) plus the float32 queries."""
    rng = np.random.default_rng(case["seed"])
    lens = rng.integers(case["lo"], case["hi"] + 1, size=case["nodes"])
    offs = np.zeros(lens.size + 1, dtype=np.uint64)
    offs[1:] = np.cumsum(lens)
    kv, hd = case["kv"], case["hd"]
    raw = rng.standard_normal(int(offs[-1]) * kv * hd).astype(np.float32)
    qs = rng.standard_normal((case["queries"], case["H"], case["Qt"], hd)
                             ).astype(np.float32)
    dt = case["dtype"]
    if dt == "f32":
        return raw, offs, None, oracle.F32, qs
    if dt == "bf16":
        return oracle.bf16_bits(raw), offs, None, oracle.BF16, oracle.round_bf16(qs)
    codes, scales = oracle.quantize_int8(raw.reshape(-1, hd), case["group"],
                                         case["scale_dtype"])
    return codes.reshape(-1), offs, scales.reshape(-1), oracle.I8, qs


def gqa_values(case: dict) -> np.ndarray:
    """The decoded (law-level) float32 key values of a case, flat."""
    keys, offs, scales, code, _ = gqa_storage(case)
    if code == oracle.F32:
        return keys
    if code == oracle.BF16:
        return oracle.bf16_to_f32(keys)
    return oracle.dequantize_int8(keys.reshape(-1, case["hd"]), scales,
                                  case["group"], case["scale_dtype"]).reshape(-1)


def gqa_inputs(case: dict):
    """Per-node decoded blocks [kv, L, hd] and float32 queries."""
    keys, offs, _, _, qs = gqa_storage(case)
    vals = gqa_values(case)
    kv, hd = case["kv"], case["hd"]
    blocks = []
    for i in range(offs.size - 1):
        a, b = int(offs[i]) * kv * hd, int(offs[i + 1]) * kv * hd
        blocks.append(vals[a:b].reshape(kv, -1, hd))
    return blocks, qs
