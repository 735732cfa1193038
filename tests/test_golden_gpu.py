"""The HIP route library against the reference router's own route orders
(tests/golden/route_goldens.json, produced by cpp/grm_runtime.cpp)."""

import json
from pathlib import Path

import numpy as np
import pytest

from graftrepository_amd import GqaNodeBank, MlaNodeBank
from graftrepository_amd.workloads import digest
from tests.golden.cases import (GQA_CASES, MLA_CASES, gqa_inputs, gqa_storage,
                                mla_inputs)

pytestmark = pytest.mark.gpu
GOLDEN = json.loads((Path(__file__).parent / "golden" / "route_goldens.json")
                    .read_text())
NO_ID = np.iinfo(np.uint64).max


def _case(kind, name):
    return next(c for c in GOLDEN[kind] if c["name"] == name)


@pytest.mark.parametrize("case", MLA_CASES, ids=[c["name"] for c in MLA_CASES])
def test_mla_library_reproduces_reference_orders(hip_lib, case):
    rows, qs = mla_inputs(case)
    gold = _case("mla", case["name"])
    assert digest(rows, qs) == gold["digest"]
    with MlaNodeBank(rows) as bank:
        res = bank.route(qs, case["topk"])
    for qi, want in enumerate(gold["ids"]):
        got = [int(x) for x in res.ids[qi] if x != NO_ID]
        assert got == want


@pytest.mark.parametrize("case", GQA_CASES, ids=[c["name"] for c in GQA_CASES])
def test_gqa_library_reproduces_reference_orders(hip_lib, case):
    blocks, qs = gqa_inputs(case)
    gold = _case("gqa", case["name"])
    keys, offs, scales, _, _ = gqa_storage(case)
    dtype = {"f32": "f32", "bf16": "bf16", "i8": "i8"}[case["dtype"]]
    kw = {}
    if dtype == "i8":
        kw = dict(scales=scales, scale_dtype=case["scale_dtype"],
                  group_size=case["group"])
    with GqaNodeBank(keys, offs, kv_heads=case["kv"], head_dim=case["hd"],
                     dtype=dtype, **kw) as bank:
        res = bank.route(qs, case["topk"])
    for qi, want in enumerate(gold["ids_fp64_law"]):
        got = [int(x) for x in res.ids[qi] if x != NO_ID]
        assert got == want
