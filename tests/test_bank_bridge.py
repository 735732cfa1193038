"""Arena bridge logic on the CPU: walk laws, deltas, the epoch gate and the
exclude-aware route order.

The walks follow core/graft_arena.py:1124-1162 (MLA) and :2933-2977 (GQA).
The route order follows :1282-1364.  The bank behind the bridge here is an
in-memory row store routed by the oracle, so every case runs without a GPU.
The GPU file drives the same bridge over real device banks.
"""

import numpy as np
import pytest

import oracle
from graftrepository_amd import bank_bridge as bb

NO_ID = np.iinfo(np.uint64).max


class _RowStore:
    """Stands in for a device bank: node id -> row."""

    def __init__(self, node_ids, rows):
        self.rows = {int(n): np.asarray(r, np.float32) for n, r in zip(node_ids, rows)}
        self.ops = [("create", len(self.rows))]

    def close(self):
        self.rows = {}


class CpuMlaBridge(bb._Bridge):
    _full_walk = staticmethod(bb._walk_mla)

    def _create(self, node_ids, rows):
        self.bank = _RowStore(node_ids, rows)
        return len(rows)

    def _apply(self, evict_ids, append_pos, node_ids, rows):
        for nid in evict_ids:
            del self.bank.rows[int(nid)]
        for p in append_pos:
            nid = int(node_ids[p])
            assert nid not in self.bank.rows, "append of a live id"
            self.bank.rows[nid] = np.asarray(rows[p], np.float32)
        self.bank.ops.append(("delta", len(evict_ids), len(append_pos)))
        return len(append_pos), False

    def _create_side(self, keys):
        self.side = _RowStore(range(len(keys)), keys)
        return len(keys)

    def _route_main(self, query, topk):
        ids = np.asarray(sorted(self.bank.rows), dtype=np.uint64)
        rows = np.stack([self.bank.rows[int(i)] for i in ids])
        got, sc, _ = oracle.mla_route(rows, np.asarray(query, np.float32)[None],
                                      topk, node_ids=ids)
        return got[0], sc[0]

    def _score_main(self, query, node_ids):
        rows = np.stack([self.bank.rows[int(i)] for i in node_ids])
        return oracle.mla_scores(rows, np.asarray(query, np.float32)[None])[0]

    def _score_side(self, query):
        rows = np.stack([self.side.rows[i] for i in range(len(self.side.rows))])
        return oracle.mla_scores(rows, np.asarray(query, np.float32)[None])[0]


def graft(nid, cent, **kw):
    g = {"native_node_id": nid, "cent": cent}
    g.update(kw)
    return g


def test_mla_walk_law():
    rng = np.random.default_rng(1)
    c = [rng.standard_normal(8).astype(np.float32) for _ in range(4)]
    gs = [graft(10, c[0]), graft(11, c[1], retired=True),
          graft(12, c[2], kind="recall"), graft(13, c[3])]
    ids, sig, rows = bb.mla_bank_walk(gs)
    assert ids.tolist() == [10, 13]
    assert sig == ((10, 8, "<f4", id(c[0])), (13, 8, "<f4", id(c[3])))
    assert np.array_equal(rows[1], c[3])
    # Each of these declines the whole bank (fail closed to the CPU path).
    assert bb.mla_bank_walk(gs + [graft(14, c[0], child_cents=[c[1]])]) is None
    assert bb.mla_bank_walk(gs + [{"cent": c[0]}]) is None
    assert bb.mla_bank_walk(gs + [{"native_node_id": 15}]) is None
    assert bb.mla_bank_walk(gs + [graft(16, np.zeros(9, np.float32))]) is None
    assert bb.mla_bank_walk([graft(1, c[0], retired=True)]) is None
    # A retired multi-row entry is skipped before the hierarchy check.
    assert bb.mla_bank_walk(gs + [graft(17, c[0], child_cents=[1], retired=True)]) is not None


def test_gqa_walk_law():
    rng = np.random.default_rng(2)
    k1 = rng.standard_normal((2, 5, 4)).astype(np.float32)
    k2 = rng.standard_normal((2, 9, 4)).astype(np.float32)
    ids, sig, rows = bb.gqa_bank_walk([graft(1, k1), graft(2, k2)])
    assert ids.tolist() == [1, 2] and sig[1] == (2, (2, 9, 4), "<f4", id(k2))
    bad = k2.copy()
    bad[0, 3, 1] = np.inf
    assert bb.gqa_bank_walk([graft(1, k1), graft(2, bad)]) is None
    assert bb.gqa_bank_walk([graft(1, k1), graft(2, np.zeros((3, 5, 4)))]) is None
    assert bb.gqa_bank_walk([graft(1, k1), graft(2, np.zeros((2, 5, 8)))]) is None
    assert bb.gqa_bank_walk([graft(1, k1), graft(2, np.zeros((2, 0, 4)))]) is None
    assert bb.gqa_bank_walk([graft(1, k1.reshape(-1))]) is None


def rowset(nids, cids, ext):
    return bb.RowSet(np.asarray(nids, np.uint64), np.asarray(cids, np.int64),
                     np.asarray(ext, np.int64))


def test_plan_delta():
    old = rowset([1, 2, 3], [101, 102, 103], [8, 8, 8])
    ev, ap = bb.plan_delta(old, rowset([1, 3, 4], [101, 203, 104], [8, 8, 8]))
    assert sorted(ev.tolist()) == [2, 3] and ap.tolist() == [1, 2]
    ev, ap = bb.plan_delta(old, rowset([3, 2, 1], [103, 102, 101], [8, 8, 8]))
    assert ev.size == 0 and ap.size == 0
    ev, ap = bb.plan_delta(old, rowset([1, 2, 3], [101, 102, 103], [8, 9, 8]))
    assert ev.tolist() == [2] and ap.tolist() == [1]       # extent changed
    ev, ap = bb.plan_delta(None, rowset([7, 8], [1, 2], [4, 4]))
    assert ev.size == 0 and ap.tolist() == [0, 1]
    with pytest.raises(ValueError):
        bb.plan_delta(None, rowset([7, 7], [1, 2], [4, 4]))


class NoWalk(list):
    def __iter__(self):
        raise AssertionError("walked the grafts under an unchanged epoch")


def test_epoch_gate_and_events():
    rng = np.random.default_rng(3)
    gs = [graft(100 + i, rng.standard_normal(6).astype(np.float32)) for i in range(20)]
    br = CpuMlaBridge()
    ev = br.refresh(gs, 1)
    assert ev["status"] == "created" and ev["node_count"] == 20
    assert br.refresh(NoWalk(gs), 1)["status"] == "reused"
    gs[4]["note"] = "metadata only"
    assert br.refresh(gs, 2)["status"] == "signature_reused"
    gs[5]["retired"] = True
    gs.append(graft(500, rng.standard_normal(6).astype(np.float32)))
    gs[7]["cent"] = rng.standard_normal(6).astype(np.float32)
    ev = br.refresh(gs, 3)
    assert ev["status"] == "updated" and ev["evicted"] == 2 and ev["appended"] == 2
    # a digest node: served beside the bank (its keys in the side store)
    gs.append(graft(600, gs[0]["cent"], child_cents=[gs[1]["cent"]]))
    ev = br.refresh(gs, 4)
    assert ev["status"] == "updated" and ev["digest_nodes"] == 1 and ev["digest_keys"] == 2
    assert br.refresh(NoWalk(gs), 4)["status"] == "reused"
    assert br.route_order(gs[0]["cent"], 3) is not None
    gs[-1]["note"] = "metadata only"
    assert br.refresh(gs, 5)["status"] == "signature_reused"
    gs.pop()
    ev = br.refresh(gs, 6)
    assert ev["status"] == "updated" and ev["digest_nodes"] == 0 and br.side is None
    gs.append(graft(700, np.full(7, 1.0, np.float32)))  # a dim the bank cannot hold
    assert br.refresh(gs, 7)["status"] == "ineligible"
    assert br.refresh(NoWalk(gs), 7)["status"] == "ineligible_reused"
    assert br.route_order(gs[0]["cent"], 3) is None
    gs.pop()
    ev = br.refresh(gs, 8)
    assert ev["status"] == "signature_reused"
    assert sorted(br.bank.rows) == sorted(int(g["native_node_id"]) for g in gs
                                          if not g.get("retired"))


def test_random_mutations_keep_the_rows_in_step():
    rng = np.random.default_rng(4)
    gs = [graft(i, rng.standard_normal(5).astype(np.float32)) for i in range(60)]
    nxt = 60
    br = CpuMlaBridge()
    br.refresh(gs, 0)
    for epoch in range(1, 80):
        for _ in range(rng.integers(0, 6)):
            op = rng.integers(0, 4)
            live = [g for g in gs if not g.get("retired")]
            if op == 0 and len(live) > 10:
                live[rng.integers(len(live))]["retired"] = True
            elif op == 1:
                gs.append(graft(nxt, rng.standard_normal(5).astype(np.float32)))
                nxt += 1
            elif op == 2 and live:
                live[rng.integers(len(live))]["cent"] = rng.standard_normal(5).astype(np.float32)
            elif live:
                live[rng.integers(len(live))]["kind"] = "turn"  # metadata only
        br.refresh(gs, epoch)
        want = {int(g["native_node_id"]): g["cent"] for g in gs if not g.get("retired")}
        assert sorted(br.bank.rows) == sorted(want)
        for nid, row in want.items():
            assert np.array_equal(br.bank.rows[nid], row)
    assert br.bank.ops[0] == ("create", 60) and len(br.bank.ops) > 1


def test_route_order_with_excludes():
    rng = np.random.default_rng(5)
    gs = [graft(1000 - i, rng.standard_normal(12).astype(np.float32)) for i in range(40)]
    gs[3]["retired"] = True
    gs[9]["kind"] = "recall"
    br = CpuMlaBridge()
    br.refresh(gs, 1)
    q = rng.standard_normal(12).astype(np.float32)
    elig = [i for i, g in enumerate(gs) if not g.get("retired") and g.get("kind") != "recall"]
    rows = np.stack([gs[i]["cent"] for i in elig])
    ids = np.asarray([gs[i]["native_node_id"] for i in elig], np.uint64)
    full, _, _ = oracle.mla_route(rows, q[None], 16, node_ids=ids)
    by_id = {int(gs[i]["native_node_id"]): i for i in elig}
    order = [by_id[int(n)] for n in full[0]]
    assert br.route_order(q, 5) == order[:5]
    excl = {order[0], order[2], 3, 9}            # two in the bank, two not
    assert br.route_order(q, 5, exclude=excl) == [i for i in order if i not in excl][:5]
    size = len(elig)
    assert br.route_order(q, 5, exclude=excl, cand_count=size - 2) is not None
    assert br.route_order(q, 5, exclude=excl, cand_count=size) is None
    assert br.route_order(q, 0) == []
    # 16 wanted with 2 excludes in the bank: the capped ask (16) holds the
    # excluded rows, so too few survive and the caller falls back.
    assert br.route_order(q, 16, exclude={order[0], order[1]}) is None


def test_failed_update_fails_closed_and_retries_from_scratch():
    # An error part-way through applying a delta (here the append, after
    # the evictions ran) must not leave a route on a half-updated bank, and
    # a retry at the same epoch must not take the bank as current
    # (core/graft_arena.py:1270-1281 marks the route unavailable).
    rng = np.random.default_rng(6)
    gs = [graft(i, rng.standard_normal(8).astype(np.float32)) for i in range(30)]
    br = CpuMlaBridge()
    br.refresh(gs, 1)
    q = gs[3]["cent"]
    assert br.route_order(q, 3) is not None
    gs[2]["retired"] = True
    gs.append(graft(99, rng.standard_normal(8).astype(np.float32)))

    real_apply = CpuMlaBridge._apply

    def failing_apply(self, evict_ids, append_pos, node_ids, rows):
        for nid in evict_ids:
            del self.bank.rows[int(nid)]
        raise RuntimeError("append failed")

    CpuMlaBridge._apply = failing_apply
    try:
        with pytest.raises(RuntimeError, match="append failed"):
            br.refresh(gs, 2)
    finally:
        CpuMlaBridge._apply = real_apply
    assert br.bank is None and br.bank_size == 0
    assert br.route_order(q, 3) is None
    ev = br.refresh(gs, 2)                       # same epoch: walks again
    assert ev["status"] == "created"
    want = sorted(int(g["native_node_id"]) for g in gs if not g.get("retired"))
    assert sorted(br.bank.rows) == want
    assert br.route_order(q, 3) is not None


def expected_order(gs, q, topk, *, debias=False):
    """The law's order over an arena with digest nodes, from the oracle:
    each node's best finite key score (own centroid, then child_cents;
    cpp/grm_runtime.cpp:3518-3545), optionally length-debiased
    (core/graft_arena.py:839-874), ranked score desc then node id."""
    keys, owners, nids, klen = [], [], [], []
    for g in gs:
        if g.get("retired") or g.get("kind", "turn") == "recall":
            continue
        e = len(nids)
        nids.append(int(g["native_node_id"]))
        klen.append(bb.route_key_length(g))
        for k in [g["cent"], *g.get("child_cents", ())]:
            keys.append(np.asarray(k, np.float32).reshape(-1))
            owners.append(e)
    ks = oracle.mla_scores(np.stack(keys), np.asarray(q, np.float32)[None])[0]
    sc = oracle._entry_max(ks, owners, len(nids))
    if debias:
        sc = oracle.length_debias(sc, klen)
    return oracle.rank_entries(sc, nids, topk)


def digest_arena(rng, n, dim, n_digest):
    gs = [graft(3 * n - 2 * i, rng.standard_normal(dim).astype(np.float32),
                ntok=int(rng.integers(1, 600))) for i in range(n)]
    for j in range(n_digest):
        src = [g for g in gs if not g.get("retired") and "child_cents" not in g][:3]
        child = []
        for g in src:
            child.append(g["cent"])
            child.extend(g.get("child_cents", ()))
            g["retired"] = True
        gs.append(graft(10_000 + j, rng.standard_normal(dim).astype(np.float32),
                        child_cents=child, kind="digest", ntok=int(rng.integers(1, 600))))
    return gs


def test_digest_walk_law():
    rng = np.random.default_rng(7)
    gs = digest_arena(rng, 12, 5, 2)
    assert bb.mla_bank_walk(gs) is None          # the reference's walk declines
    rs, rows, gidx, cents, dg, kl = bb._walk_mla(gs, True, True)
    live = [i for i, g in enumerate(gs) if not g.get("retired")]
    plain = [i for i in live if "child_cents" not in gs[i]]
    assert list(gidx) == plain and list(dg.gidx) == [i for i in live if i not in plain]
    for j, gi in enumerate(dg.gidx):
        g = gs[gi]
        want = [g["cent"], *g["child_cents"]]
        got = dg.keys[dg.offs[j]:dg.offs[j + 1]]
        assert len(got) == len(want)
        assert all(np.array_equal(a, b) for a, b in zip(got, want))
    # the second digest holds the first one's leaf keys too (generations flatten)
    assert dg.offs[2] - dg.offs[1] >= 4
    assert list(kl[0]) == [gs[i]["ntok"] for i in plain]
    assert list(kl[1]) == [gs[i]["ntok"] for i in dg.gidx]


def test_length_debias_law_closed_forms():
    # K = 1: sqrt(log2 2) = 1, the identity; K = 3: sqrt(2); K = 15: 2;
    # K <= 0 or malformed counts as 1; negative scores are multiplied
    sc = [0.5, 0.5, 0.5, -0.5, 0.5, -0.25, 0.0, 0.75]
    kl = [1, 3, 15, 15, 0, 3, 40, "x"]
    want = [0.5, 0.5 / np.sqrt(2.0), 0.25, -1.0, 0.5, -0.25 * np.sqrt(2.0), 0.0, 0.75]
    got = oracle.length_debias(sc, kl)
    np.testing.assert_array_equal(got, np.asarray(want))
    # the bridge's vectorised form equals the oracle's on random scores
    rng = np.random.default_rng(9)
    s = rng.standard_normal(2000).astype(np.float32)
    k = rng.integers(-2, 5000, size=2000)
    np.testing.assert_array_equal(bb.apply_length_debias(s, k), oracle.length_debias(s, k))
    # monotone in the score for a fixed K, and a longer key never gains
    d = oracle.length_debias(np.sort(s), np.full(2000, 37))
    assert np.all(np.diff(d) >= 0)
    pos = np.abs(s)
    assert np.all(oracle.length_debias(pos, k + 10) <= oracle.length_debias(pos, k))


def test_route_key_length_law():
    assert bb.route_key_length({"cent": np.zeros((2, 9, 4))}) == 9
    assert bb.route_key_length({"cent": np.zeros((2, 0, 4))}) == 1
    assert bb.route_key_length({"cent": np.zeros(8), "ntok": 33}) == 33
    assert bb.route_key_length({"cent": np.zeros(8)}) == 1
    assert bb.route_key_length({"cent": np.zeros(8), "ntok": "?"}) == 1
    assert bb.route_key_length({"cent": np.zeros(8), "ntok": -4}) == 1


@pytest.mark.parametrize("debias", [False, True])
def test_digest_and_debias_routes_follow_the_law(debias):
    rng = np.random.default_rng(8 + debias)
    dim = 6
    gs = digest_arena(rng, 40, dim, 3)
    br = CpuMlaBridge(length_debias=debias)
    for epoch in range(6):
        if epoch:
            live = [g for g in gs if not g.get("retired")]
            live[int(rng.integers(len(live)))]["retired"] = True
            gs.append(graft(20_000 + epoch, rng.standard_normal(dim).astype(np.float32),
                            ntok=int(rng.integers(1, 600))))
            if epoch % 2:
                d = [g for g in gs if "child_cents" in g and not g.get("retired")][0]
                d["child_cents"] = d["child_cents"] + [rng.standard_normal(dim).astype(np.float32)]
        br.refresh(gs, epoch)
        for _ in range(3):
            q = rng.standard_normal(dim).astype(np.float32)
            ids, sc = br.route_scored(q, 9)
            w_ids, w_sc = expected_order(gs, q, 9, debias=debias)
            np.testing.assert_array_equal(ids, w_ids)
            np.testing.assert_array_equal(sc, w_sc)


def test_route_receipts_follow_the_route_profile(monkeypatch):
    # core/graft_arena.py:161-256: a receipt per profiled route (phase
    # times, the bank's event, fallback reasons, the ranking's prefix);
    # none for an unprofiled route
    monkeypatch.delenv("GRM_ROUTE_SEAMS_PROFILE", raising=False)
    rng = np.random.default_rng(17)
    gs = [graft(300 + i, rng.standard_normal(8).astype(np.float32)) for i in range(30)]
    q = rng.standard_normal(8).astype(np.float32)
    br = CpuMlaBridge()
    br.refresh(gs, 1)
    want = br.route_order(q, 5)
    assert want is not None and br.last_route_receipt is None
    assert br.route_receipt_history == []

    monkeypatch.setenv("GRM_ROUTE_SEAMS_PROFILE", "on")
    gs[2]["cent"] = rng.standard_normal(8).astype(np.float32)
    br.refresh(gs, 2)
    got = br.route_order(q, 5)
    r = br.last_route_receipt
    assert r["schema"] == bb.ROUTE_RECEIPT_SCHEMA and r["epoch"] == 2
    assert r["route_backend"] == "hip" and r["fallbacks"] == []
    assert r["rebuilds"]["device_bank"]["status"] == "updated"
    assert r["ranking_count"] == 5 and r["ranking_prefix"] == got
    assert r["candidate_count"] == 30
    t = r["terms_ms"]
    for name in ("bank_refresh_ms", "device_route_call_ms", "ranking_ms",
                 "result_remap_ms", "route_wall_ms"):
        assert t[name] >= 0.0, name
    assert t["bank_refresh_ms"] > 0.0
    assert t["route_wall_ms"] >= t["device_route_call_ms"]
    # the refresh time goes to the next route only
    br.route_order(q, 5)
    assert br.last_route_receipt["terms_ms"]["bank_refresh_ms"] == 0.0
    assert len(br.route_receipt_history) == 2

    # fallbacks, each with its reason
    assert br.route_order(q, None) is None
    assert br.last_route_receipt["fallbacks"] == ["requires_limited_route"]
    assert br.last_route_receipt["route_backend"] is None
    assert br.route_order(q, 5, cand_count=7) is None
    assert br.last_route_receipt["fallbacks"] == ["candidate_subset_mismatch"]
    order = br.route_order(q, 16)
    assert br.route_order(q, 16, exclude={order[0], order[1]}) is None
    assert br.last_route_receipt["fallbacks"] == ["short_result"]
    gs.append(graft(999, np.full(9, 1.0, np.float32)))  # a dim the bank cannot hold
    br.refresh(gs, 3)
    assert br.route_order(q, 5) is None
    assert br.last_route_receipt["fallbacks"] == ["bank_ineligible"]
    assert br.last_route_receipt["rebuilds"]["device_bank"]["status"] == "ineligible"

    # the constructor flag asks for receipts without the environment
    monkeypatch.delenv("GRM_ROUTE_SEAMS_PROFILE")
    gs.pop()
    br2 = CpuMlaBridge(route_profile=True, length_debias=True)
    gs.append(graft(800, gs[0]["cent"], child_cents=[gs[1]["cent"]]))
    br2.refresh(gs, 1)
    assert br2.route_order(q, 4) is not None
    t2 = br2.last_route_receipt["terms_ms"]
    assert "device_score_all_ms" in t2 and "device_digest_score_ms" in t2
