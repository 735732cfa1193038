"""Routes completed through host-mapped flags never merge an earlier route's lists.

Untimed routes, and timed routes on the device clock, hand each block's
top-k list to the host through host-mapped memory and signal it with a
per-block completion flag.  The host can see a block's flag before that
block's list stores, so every list entry carries the route's tag and the
host waits for all tags (store_entry / wait_tagged in grm_common).  Here
two queries whose answers differ in every block alternate thousands of
times on a bank spread over several finalize (GQA) or route (MLA)
blocks; a list left over from the other query would change the ids, so
every result must equal the oracle's for its own query.
"""

import numpy as np
import pytest

import oracle
from graftrepository_amd import GqaNodeBank, MlaNodeBank

pytestmark = pytest.mark.gpu
NO_ID = np.iinfo(np.uint64).max


def assert_same(res_ids, res_scores, want_ids, want_scores):
    np.testing.assert_array_equal(res_ids, want_ids)
    filled = want_ids != NO_ID
    np.testing.assert_array_equal(res_scores[filled].view(np.uint32),
                                  want_scores[filled].view(np.uint32))


@pytest.mark.parametrize("timing", ["clock", "untimed"])
def test_gqa_alternating_queries_take_only_their_own_lists(hip_lib, monkeypatch, timing):
    monkeypatch.setenv("GRM_HIP_GQA_SCREEN", "1")
    monkeypatch.setenv("GRM_HIP_GQA_BOUND", "0")
    monkeypatch.delenv("GRM_HIP_ROUTE_TIMING", raising=False)
    rng = np.random.default_rng(2024)
    n, kv, hd, H = 300, 4, 128, 16  # 300 slots: five finalize blocks of 64
    lens = rng.integers(4, 40, size=n).astype(np.uint64)
    offs = np.zeros(n + 1, np.uint64)
    offs[1:] = np.cumsum(lens)
    keys = rng.standard_normal(int(offs[-1]) * kv * hd).astype(np.float32)
    qs = [rng.standard_normal((1, H, 1, hd)).astype(np.float32) for _ in range(2)]
    want = [oracle.gqa_route(oracle.bf16_bits(keys), oracle.BF16, offs, kv, hd, q, 6)[:2] for q in qs]
    assert not np.array_equal(want[0][0], want[1][0])
    timed = timing == "clock"
    with GqaNodeBank(keys, offs, kv_heads=kv, head_dim=hd, dtype="bf16") as bank:
        for i in range(3000):
            j = i & 1
            res = bank.route(qs[j], 6, timed=timed)
            assert_same(res.ids, res.scores, *want[j])
            if timed:
                assert res.device_ms > 0.0
        stats = bank.route_stats()
    assert stats["screen_refine"] >= 3000


@pytest.mark.parametrize("timing", ["clock", "untimed"])
def test_mla_alternating_queries_take_only_their_own_lists(hip_lib, monkeypatch, timing):
    monkeypatch.delenv("GRM_HIP_ROUTE_TIMING", raising=False)
    rng = np.random.default_rng(2025)
    rows = rng.standard_normal((40_000, 288)).astype(np.float32)
    qs = [rng.standard_normal((1, 288)).astype(np.float32) for _ in range(2)]
    want = [oracle.mla_route(rows, q, 8)[:2] for q in qs]
    assert not np.array_equal(want[0][0], want[1][0])
    timed = timing == "clock"
    with MlaNodeBank(rows) as bank:
        for i in range(3000):
            j = i & 1
            res = bank.route(qs[j], 8, timed=timed)
            assert_same(res.ids, res.scores, *want[j])
            if timed:
                assert res.device_ms > 0.0
