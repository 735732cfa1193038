"""fp32 GQA banks on the matrix-core screens: the fp16 key copy.

The reference hands its GQA router a dense, zero-padded fp32 bank
(core/graft_arena.py:2979-3042, core/grm_cuda_router.py:44;
grm_gqa_cuda_arena_create, cpp/grm_runtime_c.h).  The library keeps an
fp16 copy of an fp32 bank's keys beside the fp32 rows: the screens read
the copy with its rounding in their bound, every exact recomputation reads
the fp32 rows, so ids and score bits stay the law's
(cpp/grm_runtime.cpp:2980-3029).  Dense banks drop their trailing
all-zero tokens (|q.0| = 0 never raises a maximum that starts at 0; one
token always stays).  Every case is checked against the oracle.
"""

import ctypes

import numpy as np
import pytest

import oracle
from graftrepository_amd import GqaNodeBank
from graftrepository_amd.grm_hip_router import CudaGQARouteSidecar

pytestmark = pytest.mark.gpu
NO_ID = np.iinfo(np.uint64).max


def assert_same(res_ids, res_scores, want_ids, want_scores):
    np.testing.assert_array_equal(res_ids, want_ids)
    filled = want_ids != NO_ID
    if res_scores is not None:
        assert np.all(np.isnan(res_scores[~filled]))
        np.testing.assert_array_equal(res_scores[filled].view(np.uint32),
                                      want_scores[filled].view(np.uint32))


def ragged_f32(rng, n, kv, hd, lo, hi):
    lens = rng.integers(lo, hi + 1, size=n).astype(np.uint64)
    offs = np.zeros(n + 1, np.uint64)
    offs[1:] = np.cumsum(lens)
    keys = rng.standard_normal(int(offs[-1]) * kv * hd).astype(np.float32)
    return keys, offs


def set_mode(monkeypatch, mode):
    monkeypatch.setenv("GRM_HIP_GQA_SCREEN", "0" if mode == "exact" else "1")
    monkeypatch.setenv("GRM_HIP_GQA_BOUND", "1" if mode == "bv" else "0")


@pytest.mark.parametrize("mode", ["sr", "bv", "exact"])
@pytest.mark.parametrize("hd,Qt", [(128, 1), (128, 4), (64, 3), (256, 2)])
def test_f32_bank_through_the_fp16_copy(hip_lib, monkeypatch, mode, hd, Qt):
    set_mode(monkeypatch, mode)
    rng = np.random.default_rng(hd * 10 + Qt)
    kv, H = 4, 16
    keys, offs = ragged_f32(rng, 240, kv, hd, 1, 300)
    qs = rng.standard_normal((3, H, Qt, hd)).astype(np.float32)
    with GqaNodeBank(keys, offs, kv_heads=kv, head_dim=hd) as bank:
        res = bank.route(qs, 5)
        stats = bank.route_stats()
    ids, sc, _ = oracle.gqa_route(keys, oracle.F32, offs, kv, hd, qs, 5)
    assert_same(res.ids, res.scores, ids, sc)
    if mode == "sr":
        assert stats["screen_refine"] > 0 and stats["exact"] == 0
    elif mode == "bv":
        assert stats["bound_verify"] > 0 and stats["exact"] == 0
    else:
        assert stats["exact"] == 3


@pytest.mark.parametrize("mode", ["sr", "bv"])
def test_f32_values_outside_the_fp16_range(hip_lib, monkeypatch, mode):
    # nodes whose keys overflow fp16 (|k| >= 65520) are recomputed exactly;
    # values under the fp16 normal range round with an absolute error
    set_mode(monkeypatch, mode)
    rng = np.random.default_rng(404)
    kv, hd, H, Qt = 2, 128, 8, 2
    keys, offs = ragged_f32(rng, 120, kv, hd, 1, 40)
    blocks = []
    for i in range(120):
        b = keys[int(offs[i]) * kv * hd:int(offs[i + 1]) * kv * hd].copy()
        f = i % 5
        if f == 1:
            b *= np.float32(3.0e4)          # straddles the fp16 maximum
        elif f == 2:
            b *= np.float32(2.0 ** -20)     # fp16 subnormal range
        elif f == 3:
            b[::97] = np.float32(1.0e30)    # a few huge values
        elif f == 4:
            b *= np.float32(2.0 ** -30)     # flushed to zero in fp16
        blocks.append(b)
    keys = np.concatenate(blocks)
    qs = rng.standard_normal((4, H, Qt, hd)).astype(np.float32)
    qs[1] *= np.float32(2.0 ** 20)
    qs[2] *= np.float32(2.0 ** -20)
    with GqaNodeBank(keys, offs, kv_heads=kv, head_dim=hd) as bank:
        res = bank.route(qs, 8)
    ids, sc, _ = oracle.gqa_route(keys, oracle.F32, offs, kv, hd, qs, 8)
    assert_same(res.ids, res.scores, ids, sc)


def test_f32_copy_follows_append_evict_compact(hip_lib, monkeypatch):
    set_mode(monkeypatch, "sr")
    rng = np.random.default_rng(505)
    kv, hd, H = 4, 128, 16
    keys, offs = ragged_f32(rng, 60, kv, hd, 1, 80)
    ids0 = np.arange(60, dtype=np.uint64) + 1
    blocks = {int(i): keys[int(offs[j]) * kv * hd:int(offs[j + 1]) * kv * hd]
              for j, i in enumerate(ids0)}
    q = rng.standard_normal((2, H, 3, hd)).astype(np.float32)
    with GqaNodeBank(keys, offs, kv_heads=kv, head_dim=hd, node_ids=ids0,
                     capacity_nodes=120, capacity_tokens=20000) as bank:
        for step in range(3):
            ev = rng.choice(sorted(blocks), size=8, replace=False)
            bank.evict(ev)
            for i in ev.tolist():
                del blocks[i]
            lens = rng.integers(1, 90, size=10)
            new = [rng.standard_normal(int(L) * kv * hd).astype(np.float32) for L in lens]
            nid = np.arange(10, dtype=np.uint64) + 1000 + 100 * step
            bank.append(np.concatenate(new), lens.astype(np.uint64), nid)
            for i, b in zip(nid.tolist(), new):
                blocks[i] = b
            if step == 1:
                bank.compact()
            order = sorted(blocks)
            cat = np.concatenate([blocks[i] for i in order])
            o = np.zeros(len(order) + 1, np.uint64)
            o[1:] = np.cumsum([blocks[i].size // (kv * hd) for i in order])
            res = bank.route(q, 4)
            want, wsc, _ = oracle.gqa_route(cat, oracle.F32, o, kv, hd, q, 4,
                                            node_ids=np.array(order, dtype=np.uint64))
            assert_same(res.ids, res.scores, want, wsc)


@pytest.mark.parametrize("Qt", [1, 4, 9])
def test_dense_padded_bank_surface(hip_lib, Qt):
    # the reference's dense bank: [nodes, kv, key_tokens, hd], zero tails;
    # one node is all zeros, one has no padding, one keeps an interior zero
    # token ahead of real ones
    rng = np.random.default_rng(600 + Qt)
    n, kv, T, hd, H = 96, 8, 64, 128, 32
    bank_np = rng.standard_normal((n, kv, T, hd)).astype(np.float32)
    lens = rng.integers(1, T + 1, size=n)
    lens[5] = T
    for i in range(n):
        bank_np[i, :, lens[i]:, :] = 0.0
    bank_np[7] = 0.0
    bank_np[9, :, 3, :] = -0.0
    qs = rng.standard_normal((3, H, Qt, hd)).astype(np.float32)
    node_ids = np.arange(n, dtype=np.uint64) * 3 + 11
    sidecar = CudaGQARouteSidecar.build()
    bank = sidecar.create_bank(bank_np, node_ids)
    mapped, receipt = bank.route_topk(qs, topk=5, warmup=1)
    offs = np.arange(n + 1, dtype=np.uint64) * T
    want, _, _ = oracle.gqa_route(bank_np.reshape(-1), oracle.F32, offs, kv, hd, qs, 5)
    np.testing.assert_array_equal(mapped, node_ids[want])
    assert receipt.measured_queries == 2
    bank.close()


def test_dense_padded_bank_trims_and_keeps_the_nan_law(hip_lib):
    # trailing zero tokens are not placed, but an all-zero node keeps one
    # token: against a query holding NaN it scores NaN, as the law does
    rng = np.random.default_rng(611)
    n, kv, T, hd, H = 20, 2, 32, 64, 4
    bank_np = rng.standard_normal((n, kv, T, hd)).astype(np.float32)
    bank_np[:, :, 10:, :] = 0.0
    bank_np[3] = 0.0
    keys_ptr = np.ascontiguousarray(bank_np)
    lib = hip_lib
    arena = ctypes.c_void_p()
    rc = lib.grm_gqa_cuda_arena_create(keys_ptr.ctypes.data, n, kv, T, hd, ctypes.byref(arena))
    assert rc == 0
    info = np.zeros(8, dtype=np.uint64)
    assert lib.grm_gqa_hip_bank_info(arena, info.ctypes.data) == 0
    # 19 nodes of 10 tokens and one of 1, each padded to 8-token rows
    assert int(info[2]) == 19 * 16 + 8
    q = rng.standard_normal((1, H, 1, hd)).astype(np.float32)
    q[0, 1, 0, 5] = np.nan
    out = np.zeros(3, dtype=np.uint64)
    ms = ctypes.c_float()
    assert lib.grm_gqa_cuda_arena_route(arena, q.ctypes.data, 1, H, 1, 0, 3, out.ctypes.data,
                                        ctypes.addressof(ms)) == 0
    offs = np.arange(n + 1, dtype=np.uint64) * T
    want, _, _ = oracle.gqa_route(bank_np.reshape(-1), oracle.F32, offs, kv, hd, q, 3)
    np.testing.assert_array_equal(out, want[0])
    assert np.all(out == NO_ID)
    assert lib.grm_gqa_cuda_arena_destroy(arena) == 0
