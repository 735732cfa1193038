"""Arena bridges over device banks: after every refresh the bank answers as
a bank built from scratch over the arena's current rows.

That is checked against the oracle, bit-exact in ids and scores.  Mutation
sequences retire, add, replace and touch (metadata only) grafts between
epochs, as the arena's mutation sites do (core/graft_arena.py:278-291).
The bridges start with no headroom, so their capacity-growth path runs;
the GQA bank also compacts its token arena.
"""

import numpy as np
import pytest

import oracle
from graftrepository_amd import GqaRouteBankBridge, MlaRouteBankBridge

pytestmark = pytest.mark.gpu
NO_ID = np.iinfo(np.uint64).max


def assert_same(res, want_ids, want_scores):
    np.testing.assert_array_equal(res.ids, want_ids)
    filled = want_ids != NO_ID
    np.testing.assert_array_equal(res.scores[filled].view(np.uint32),
                                  want_scores[filled].view(np.uint32))


def mutate(rng, gs, make, nxt, n_ops):
    for _ in range(n_ops):
        op = int(rng.integers(0, 4))
        live = [g for g in gs if not g.get("retired")]
        if op == 0 and len(live) > 20:
            live[int(rng.integers(len(live)))]["retired"] = True
        elif op == 1:
            gs.append({"native_node_id": nxt, "cent": make()})
            nxt += 1
        elif op == 2 and live:
            live[int(rng.integers(len(live)))]["cent"] = make()
        elif live:
            live[int(rng.integers(len(live)))]["touched"] = True
    return nxt


def current(gs):
    return [g for g in gs if not g.get("retired")]


def test_mla_bridge_follows_the_arena(hip_lib):
    rng = np.random.default_rng(21)
    dim = 96
    make = lambda: rng.standard_normal(dim).astype(np.float32)
    gs = [{"native_node_id": 5000 - i, "cent": make()} for i in range(3000)]
    nxt = 10_000
    statuses = set()
    with MlaRouteBankBridge(headroom=1.0) as br:
        for epoch in range(25):
            if epoch:
                nxt = mutate(rng, gs, make, nxt, int(rng.integers(0, 40)))
            statuses.add(br.refresh(gs, epoch)["status"])
            live = current(gs)
            rows = np.stack([g["cent"] for g in live])
            ids = np.asarray([g["native_node_id"] for g in live], np.uint64)
            q = rng.standard_normal((3, dim)).astype(np.float32)
            q[1] = live[int(rng.integers(len(live)))]["cent"]   # an exact match
            res = br.bank.route(q, 8)
            want_ids, want_sc, _ = oracle.mla_route(rows, q, 8, node_ids=ids)
            assert_same(res, want_ids, want_sc)
            assert br.bank.info()["live"] == len(live)
        assert br.refresh(gs, 24)["status"] == "reused"
    assert {"created", "updated", "rebuilt"} <= statuses, statuses


def test_mla_bridge_route_order_excludes(hip_lib):
    rng = np.random.default_rng(22)
    gs = [{"native_node_id": 7 * i + 3, "cent": rng.standard_normal(64).astype(np.float32)}
          for i in range(500)]
    gs[10]["retired"] = True
    with MlaRouteBankBridge() as br:
        br.refresh(gs, 1)
        q = rng.standard_normal(64).astype(np.float32)
        live_idx = [i for i, g in enumerate(gs) if not g.get("retired")]
        rows = np.stack([gs[i]["cent"] for i in live_idx])
        ids = np.asarray([gs[i]["native_node_id"] for i in live_idx], np.uint64)
        full, _, _ = oracle.mla_route(rows, q[None], 16, node_ids=ids)
        by_id = {int(gs[i]["native_node_id"]): i for i in live_idx}
        order = [by_id[int(n)] for n in full[0]]
        assert br.route_order(q, 6) == order[:6]
        excl = {order[1], order[3], 10}
        assert br.route_order(q, 6, exclude=excl) == [i for i in order if i not in excl][:6]


def test_gqa_bridge_follows_the_arena(hip_lib):
    rng = np.random.default_rng(23)
    kv, hd = 2, 64
    make = lambda: rng.standard_normal((kv, int(rng.integers(1, 48)), hd)).astype(np.float32)
    gs = [{"native_node_id": 900 - i, "cent": make()} for i in range(150)]
    nxt = 2000
    statuses = set()
    with GqaRouteBankBridge(headroom=1.0) as br:
        for epoch in range(20):
            if epoch:
                nxt = mutate(rng, gs, make, nxt, int(rng.integers(0, 20)))
            statuses.add(br.refresh(gs, epoch)["status"])
            live = current(gs)
            keys = np.concatenate([g["cent"].reshape(-1) for g in live])
            lens = np.asarray([g["cent"].shape[1] for g in live], np.uint64)
            offs = np.zeros(len(live) + 1, np.uint64)
            offs[1:] = np.cumsum(lens)
            ids = np.asarray([g["native_node_id"] for g in live], np.uint64)
            q = rng.standard_normal((2, 4 * kv, 1, hd)).astype(np.float32)
            res = br.bank.route(q, 5)
            want_ids, want_sc, _ = oracle.gqa_route(keys, oracle.F32, offs, kv, hd, q, 5,
                                                    node_ids=ids)
            assert_same(res, want_ids, want_sc)
            assert br.bank.info()["live"] == len(live)
    assert {"created", "updated"} <= statuses, statuses
