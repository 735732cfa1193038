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


class _NoComputeLib:
    """Stands in for the library: any route call is a test failure."""

    def __getattr__(self, name):
        if "route" in name:
            raise AssertionError(f"{name} called with bad arguments")
        return lambda *a: 0


def _bank_without_device(cls, **attrs):
    import ctypes
    b = cls.__new__(cls)
    b._lib = _NoComputeLib()
    b._h = ctypes.c_void_p(1)
    for k, v in attrs.items():
        setattr(b, k, v)
    return b


def test_device_query_shapes_are_checked_before_the_call():
    from graftrepository_amd.node_bank import GqaNodeBank, MlaNodeBank

    class Dev:  # a device buffer that states its size
        def __init__(self, nbytes):
            self.nbytes = nbytes

        def data_ptr(self):
            return 0x1000

    g = _bank_without_device(GqaNodeBank, head_dim=128, dtype=0)
    with pytest.raises(ValueError, match="head_dim"):
        g.route(Dev(1 << 20), 3, on_device=True, query_shape=(1, 32, 1, 64))
    with pytest.raises(ValueError, match="bytes"):
        g.route(Dev(32 * 128 * 4 - 4), 3, on_device=True, query_shape=(1, 32, 1, 128))
    with pytest.raises(ValueError, match="bytes"):
        g.route(Dev(2 * 32 * 4 * 128 * 2 - 2), 3, on_device=True, query_dtype="bf16",
                query_shape=(2, 32, 4, 128))
    m = _bank_without_device(MlaNodeBank, dim=288, dtype=0)
    with pytest.raises(ValueError, match="bytes"):
        m.route(Dev(288 * 4 * 3 - 4), 3, on_device=True, query_count=3)


class _RecordingLib:
    """Records each C call's arguments and returns 0 (no device work)."""

    def __init__(self):
        self.calls = []

    def __getattr__(self, name):
        def fn(*args):
            self.calls.append((name, args))
            if name.endswith(("_create", "_upload_queries")):
                args[-1]._obj.value = 0x1000   # the handle out-parameter
            return 0
        return fn


@pytest.mark.parametrize("mod", ["mla_probe", "gqa_probe"])
def test_probe_layer_argument_order(monkeypatch, mod):
    import importlib

    from graftrepository_amd import _lib, probe
    m = importlib.import_module(f"graftrepository_amd.{mod}")
    fake = _RecordingLib()
    monkeypatch.setattr(probe._lib, "load", lambda path=None: fake)
    gqa = mod == "gqa_probe"
    bank = np.zeros((5, 2, 7, 16) if gqa else (5, 16), np.float32)
    qs = np.zeros((3, 8, 4, 16) if gqa else (3, 16), np.float32)
    p = m.HipProbe()
    assert m.CudaProbe is m.HipProbe
    ids, ms, wall = p.route_topk(bank, qs, warmup=1, topk=2)
    assert ids.shape == (3, 2) and ids.dtype == np.uint64 and wall >= 0.0
    arena = p.create_arena(bank)
    arena.route_topk(qs, warmup=1, topk=2)
    dq = p.upload_queries(qs)
    arena.route_topk_device(dq, warmup=0, topk=2)
    pre = "grm_gqa" if gqa else "grm_mla"
    names = [c[0] for c in fake.calls]
    assert names == [f"{pre}_cublas_route", f"{pre}_cuda_arena_create",
                     f"{pre}_cuda_arena_route", f"{pre}_cuda_upload_queries",
                     f"{pre}_cuda_arena_route_device"]
    for name, args in fake.calls:
        assert len(args) == len(_lib.SIGNATURES[name][1]), name
    ints = [a for a in fake.calls[0][1] if isinstance(a, int)]
    if gqa:   # keys, q, nodes, kv, T, Q, H, Qt, hd, warmup, topk, out, ms
        assert fake.calls[0][1][2:11] == (5, 2, 7, 3, 8, 4, 16, 1, 2)
        assert fake.calls[2][1][2:7] == (3, 8, 4, 1, 2)
        assert (arena.nodes, arena.kv_heads, arena.key_tokens, arena.head_dim) == (5, 2, 7, 16)
    else:     # rows, q, nodes, dim, Q, warmup, topk, out, ms
        assert fake.calls[0][1][2:7] == (5, 16, 3, 1, 2)
        assert fake.calls[2][1][2:6] == (3, 16, 1, 2)
        assert (arena.nodes, arena.dim) == (5, 16)
    assert ints
    with pytest.raises(ValueError):
        arena.route_topk(qs[..., :8], warmup=0, topk=2)
    with pytest.raises(ValueError):
        arena.route_topk(qs, warmup=0, topk=6)
    arena.close()
    with pytest.raises(RuntimeError, match="closed"):
        arena.route_topk(qs, warmup=0, topk=2)
    dq.close()
    assert names.count(f"{pre}_cuda_free_device_ptr") == 0
    assert fake.calls[-1][0] == f"{pre}_cuda_free_device_ptr"
