"""Arena bridges over device banks: after every refresh the bank answers as
a bank built from scratch over the arena's current rows.

That is checked against the oracle, bit-exact in ids and scores.  Mutation
sequences retire, add, replace and touch (metadata only) grafts between
epochs, as the arena's mutation sites do (core/graft_arena.py:278-291).
The bridges start with no headroom, so their capacity-growth path runs;
the GQA bank also compacts its token arena.

Arenas with digest nodes (child_cents: the best of the node's own key and
its children's, core/graft_arena.py:803-811) and the length-debiased score
(:839-874) are routed through the bridge and checked per epoch against the
oracle's multi-key law, debias law and tie order.
"""

import numpy as np
import pytest

import oracle
from graftrepository_amd import GqaRouteBankBridge, MlaRouteBankBridge
from graftrepository_amd import bank_bridge as bb

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


def law_order(gs, score_keys, q, topk, debias):
    """Oracle order over the arena's live nodes: best finite key score per
    node (own key, then child_cents), optionally length-debiased, ranked
    score desc then node id."""
    keys, owners, nids, klen = [], [], [], []
    for g in gs:
        if g.get("retired") or g.get("kind", "turn") == "recall":
            continue
        e = len(nids)
        nids.append(int(g["native_node_id"]))
        klen.append(bb.route_key_length(g))
        for k in [g["cent"], *g.get("child_cents", ())]:
            keys.append(k)
            owners.append(e)
    sc = oracle._entry_max(score_keys(keys, q), owners, len(nids))
    if debias:
        sc = oracle.length_debias(sc, klen)
    return oracle.rank_entries(sc, nids, topk)


def consolidate(rng, gs, nxt, make, ntok):
    """Retire up to three live grafts into a new digest node that carries
    their keys (core/graft_arena.py:1665-1690)."""
    src = [g for g in gs if not g.get("retired")][:3]
    child = []
    for g in src:
        child.append(g["cent"])
        child.extend(g.get("child_cents", ()))
        g["retired"] = True
    gs.append({"native_node_id": nxt, "cent": make(), "child_cents": child,
               "kind": "digest", "ntok": ntok()})
    return nxt + 1


@pytest.mark.parametrize("debias", [False, True])
def test_mla_bridge_digests_and_debias(hip_lib, debias):
    rng = np.random.default_rng(31 + debias)
    dim = 80
    make = lambda: rng.standard_normal(dim).astype(np.float32)
    ntok = lambda: int(rng.integers(1, 2000))
    gs = [{"native_node_id": 4000 - i, "cent": make(), "ntok": ntok()} for i in range(2000)]
    nxt = 9000

    def score_keys(keys, q):
        return oracle.mla_scores(np.stack([np.asarray(k, np.float32) for k in keys]), q[None])[0]

    with MlaRouteBankBridge(headroom=1.0, length_debias=debias) as br:
        for epoch in range(12):
            if epoch:
                nxt = mutate(rng, gs, make, nxt, int(rng.integers(0, 30)))
                for g in gs[-3:]:
                    g.setdefault("ntok", ntok())
            if epoch % 3 == 1:
                nxt = consolidate(rng, gs, nxt, make, ntok)
            ev = br.refresh(gs, epoch)
            assert ev["status"] != "ineligible", ev
            for _ in range(3):
                q = make()
                if epoch % 2:
                    d = [g for g in gs if "child_cents" in g and not g.get("retired")]
                    if d:
                        q = d[-1]["child_cents"][0].copy()   # a digest's child key
                ids, sc = br.route_scored(q, 10)
                w_ids, w_sc = law_order(gs, score_keys, q, 10, debias)
                np.testing.assert_array_equal(ids, w_ids)
                np.testing.assert_array_equal(sc, w_sc)


@pytest.mark.parametrize("debias", [False, True])
def test_gqa_bridge_digests_and_debias(hip_lib, debias):
    rng = np.random.default_rng(41 + debias)
    kv, hd = 2, 64
    make = lambda: rng.standard_normal((kv, int(rng.integers(1, 40)), hd)).astype(np.float32)
    gs = [{"native_node_id": 700 - i, "cent": make()} for i in range(120)]
    nxt = 3000

    def score_keys(keys, q):
        lens = np.asarray([k.shape[1] for k in keys], np.uint64)
        offs = np.zeros(len(keys) + 1, np.uint64)
        offs[1:] = np.cumsum(lens)
        flat = np.concatenate([np.asarray(k, np.float32).reshape(-1) for k in keys])
        return oracle.gqa_scores(flat, oracle.F32, offs, kv, hd, q)[0]

    with GqaRouteBankBridge(headroom=1.0, length_debias=debias) as br:
        for epoch in range(10):
            if epoch:
                nxt = mutate(rng, gs, make, nxt, int(rng.integers(0, 12)))
            if epoch % 3 == 1:
                nxt = consolidate(rng, gs, nxt, make, lambda: 1)
            ev = br.refresh(gs, epoch)
            assert ev["status"] != "ineligible", ev
            for _ in range(2):
                q = rng.standard_normal((4 * kv, 2, hd)).astype(np.float32)
                ids, sc = br.route_scored(q, 6)
                w_ids, w_sc = law_order(gs, score_keys, q, 6, debias)
                np.testing.assert_array_equal(ids, w_ids)
                np.testing.assert_array_equal(sc, w_sc)


def test_gqa_bridge_route_receipts(hip_lib):
    # a profiled route over a device bank: the ranking is the oracle's and
    # the receipt names the device phases (core/graft_arena.py:161-256)
    rng = np.random.default_rng(25)
    kv, hd = 2, 64
    make = lambda: rng.standard_normal((kv, int(rng.integers(4, 40)), hd)).astype(np.float32)
    gs = [{"native_node_id": 100 + i, "cent": make()} for i in range(60)]
    q = rng.standard_normal((8, 2, hd)).astype(np.float32)
    with GqaRouteBankBridge(route_profile=True) as br:
        br.refresh(gs, 1)
        got = br.route_order(q, 6)
        r = br.last_route_receipt
    ids = np.asarray([g["native_node_id"] for g in gs], np.uint64)
    offs = np.zeros(len(gs) + 1, np.uint64)
    offs[1:] = np.cumsum([g["cent"].shape[1] for g in gs])
    keys = np.concatenate([g["cent"].reshape(-1) for g in gs])
    want, _, _ = oracle.gqa_route(keys, oracle.F32, offs, kv, hd, q[None], 6, node_ids=ids)
    by_id = {int(g["native_node_id"]): i for i, g in enumerate(gs)}
    assert got == [by_id[int(n)] for n in want[0]]
    assert r["route_backend"] == "hip" and r["fallbacks"] == []
    assert r["rebuilds"]["device_bank"]["status"] == "created"
    assert r["ranking_prefix"] == got
    t = r["terms_ms"]
    assert t["device_route_call_ms"] > 0.0 and t["bank_refresh_ms"] > 0.0
    assert t["route_wall_ms"] >= t["device_route_call_ms"]
