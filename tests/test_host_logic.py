"""Host-side logic of the drop-in surface and workloads (CPU only)."""

import numpy as np
import pytest

import oracle
from graftrepository_amd import workloads as wl
from graftrepository_amd.grm_hip_router import (
    CudaRouteReceipt, gqa_route_bank_signature, mla_route_bank_signature,
    validate_gqa_route_bank, validate_mla_route_bank)
from graftrepository_amd.node_bank import as_bf16_bits, bf16_bits_to_f32


def test_validate_mla_bank_contract():
    rows, ids = validate_mla_route_bank(np.ones((3, 4), np.float64))
    assert rows.dtype == np.float32 and rows.flags.c_contiguous
    assert ids.tolist() == [0, 1, 2] and ids.dtype == np.uint64
    with pytest.raises(ValueError):
        validate_mla_route_bank(np.ones(4))
    with pytest.raises(ValueError):
        validate_mla_route_bank(np.ones((0, 4)))
    with pytest.raises(ValueError):
        validate_mla_route_bank(np.ones((3, 4)), [1, 2])


def test_validate_gqa_bank_contract():
    keys, ids = validate_gqa_route_bank(np.ones((2, 1, 3, 4)), [7, 9])
    assert keys.shape == (2, 1, 3, 4) and ids.tolist() == [7, 9]
    with pytest.raises(ValueError):
        validate_gqa_route_bank(np.ones((2, 3, 4)))
    with pytest.raises(ValueError):
        validate_gqa_route_bank(np.ones((2, 1, 0, 4)))


def test_bank_signatures_are_content_hashes():
    a = np.arange(12, dtype=np.float32).reshape(3, 4)
    ids = np.arange(3, dtype=np.uint64)
    s1 = mla_route_bank_signature(a, ids)
    assert s1 == mla_route_bank_signature(a.copy(), ids.copy())
    b = a.copy()
    b[1, 1] += 1
    assert s1 != mla_route_bank_signature(b, ids)
    assert s1 != mla_route_bank_signature(a, ids + 1)
    k = np.zeros((2, 1, 2, 4), np.float32)
    assert len(gqa_route_bank_signature(k, np.arange(2, dtype=np.uint64))) == 32


def test_receipt_fields_match_reference():
    fields = list(CudaRouteReceipt.__dataclass_fields__)
    assert fields == ["device_route_ms_total", "device_route_ms_per_query",
                      "route_wall_ms", "route_wall_ms_first",
                      "route_wall_ms_min", "route_wall_ms_runs",
                      "device_route_ms_runs", "measured_queries",
                      "route_repeats"]


def test_bf16_helpers_agree_with_oracle():
    rng = np.random.default_rng(3)
    x = rng.standard_normal(50_000).astype(np.float32)
    x[:3] = [np.nan, np.inf, -0.0]
    np.testing.assert_array_equal(as_bf16_bits(x), oracle.bf16_bits(x))
    b = as_bf16_bits(x)
    np.testing.assert_array_equal(bf16_bits_to_f32(b), oracle.bf16_to_f32(b))


def test_mla_workload_rows_are_unit_norm_and_deterministic():
    rows = wl.mla_rows(1000, 288, seed=4)
    again = wl.mla_rows(1000, 288, seed=4)
    np.testing.assert_array_equal(rows, again)
    norms = np.linalg.norm(rows.astype(np.float64), axis=1)
    assert np.all(np.abs(norms - 1) < 1e-6)
    bf = wl.mla_rows(10, 288, seed=4, dtype="bf16")
    np.testing.assert_array_equal(bf, as_bf16_bits(rows[:10]))


def test_gqa_workload_shapes():
    lens = wl.gqa_lengths(512, seed=4, lo=16, hi=512)
    assert lens.min() >= 16 and lens.max() <= 512 and lens.dtype == np.uint64
    ln = wl.gqa_lengths(10_000, seed=5, kind="lognormal", median=256,
                        sigma=0.5, cap=4096)
    assert ln.min() >= 1 and ln.max() <= 4096
    assert 230 <= np.median(ln) <= 280
    keys, offs = wl.gqa_bank(lens[:8], 4, 32, seed=1)
    assert offs[0] == 0 and offs[-1] == lens[:8].sum()
    assert keys.size == int(offs[-1]) * 4 * 32 and keys.dtype == np.uint16
