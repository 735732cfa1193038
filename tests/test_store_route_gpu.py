"""The store route on the device: DeviceRouteStore against the oracle's
store law (pinned against the reference store in test_store_route.py).
Bar: node ids and fp32 route scores bit-exact.

Covered:

* lexical bonus from a small shared vocabulary, with repeated query keys;
* filters of known values, and of unknown values (the per-query
  string-match bit);
* metadata updates that keep unset fields (cpp/grm_runtime.cpp:2922-2946);
* route replacement (set_route on a live node) and clear_route;
* score ties from duplicate rows;
* entries of several route keys (none, one with a non-finite value, ties
  across entries), replaced by single keys and back, cleared.
"""

import numpy as np
import pytest

import oracle
from graftrepository_amd.store_route import DeviceRouteStore

pytestmark = pytest.mark.gpu

VOCAB = ["alpha", "beta", "gamma", "delta", "eps", "zeta", "eta", "theta", "iota", "kappa"]
META = [
    ["turn", "doc", "fact", "recall", "weird-kind", ""],
    ["conversation", "project", "global", "elsewhere", ""],
    ["volatile", "permanent", "session", ""],
    ["stable", "mutable", "odd", ""],
]
DEFAULT = ("turn", "conversation", "session", "ephemeral")


def test_device_store_route_matches_the_law(hip_lib):
    rng = np.random.default_rng(51)
    n, dim = 3000, 64
    rows = {1000 + i: rng.standard_normal(dim).astype(np.float32) for i in range(n)}
    rows[1005] = rows[1004].copy()                  # ties
    rows[1009] = rows[1004].copy()
    lex, meta = {}, {}
    with DeviceRouteStore(dim, capacity=4096) as st:
        def set_meta(nid, vals):
            st.set_route_metadata(nid, *vals)
            meta[nid] = tuple(v if v else o for v, o in zip(vals, meta[nid]))

        for nid, r in rows.items():
            lex[nid] = list(rng.choice(VOCAB, size=rng.integers(0, 4), replace=False))
            st.set_route(nid, r, "\n".join(lex[nid]))
            meta[nid] = DEFAULT
            set_meta(nid, tuple(str(rng.choice(m)) for m in META))
        for step in range(40):
            if step % 5 == 4:                       # mutations between queries
                for nid in rng.choice(list(rows), size=20, replace=False):
                    nid = int(nid)
                    op = rng.integers(0, 3)
                    if op == 0:
                        rows[nid] = rng.standard_normal(dim).astype(np.float32)
                        lex[nid] = list(rng.choice(VOCAB, size=rng.integers(0, 3), replace=False))
                        st.set_route(nid, rows[nid], lex[nid])
                    elif op == 1:
                        set_meta(nid, tuple(str(rng.choice(m)) for m in META))
                    else:
                        st.clear_route(nid)
                        del rows[nid], lex[nid], meta[nid]
            ids = np.asarray(sorted(rows), dtype=np.uint64)
            R = np.stack([rows[int(i)] for i in ids])
            q = rng.standard_normal(dim).astype(np.float32)
            if rng.random() < 0.3:
                q = rows[int(ids[4])].copy()
            qlex = list(rng.choice(VOCAB, size=rng.integers(0, 5), replace=True))
            filters = tuple([str(v) for v in rng.choice(m, size=rng.integers(0, 3), replace=False) if v]
                            if rng.random() < 0.5 else [] for m in META)
            k = int(rng.integers(1, 17))
            want_ids, want_sc = oracle.store_route(R, ids, [lex[int(i)] for i in ids],
                                                   [meta[int(i)] for i in ids], q, qlex, filters, k)
            got_ids, got_sc = st.route_scored(q, qlex, k, kinds=filters[0], scopes=filters[1],
                                              durabilities=filters[2], mutabilities=filters[3])
            assert got_ids == want_ids, (step, qlex, filters, k)
            np.testing.assert_array_equal(np.asarray(got_sc, np.float32).view(np.uint32),
                                          want_sc.view(np.uint32))
            assert st.route_filtered(q, "\n".join(qlex), *["\n".join(f) for f in filters],
                                     topk=k) == want_ids


def test_device_gqa_store_route_matches_the_law(hip_lib):
    # grm_store_route_gqa's law (route_gqa_raw, cpp/grm_runtime.cpp:4498-4881)
    # over the device store: raw order without lexical keys, normalised raw
    # plus the lexical bonus with them; filters of known and unknown values;
    # replacements, clears and metadata updates between queries.
    from graftrepository_amd.store_route import DeviceGqaRouteStore

    rng = np.random.default_rng(53)
    n, kv, hd, H = 400, 4, 64, 16
    blocks = {500 + i: rng.standard_normal((kv, int(rng.integers(0, 40)), hd)).astype(np.float32)
              for i in range(n)}
    blocks[505] = blocks[504].copy()                # ties
    lex, meta = {}, {}
    with DeviceGqaRouteStore(kv, hd, capacity_nodes=512, capacity_tokens=40_000) as st:
        ids0 = sorted(blocks)
        for nid in ids0:
            lex[nid] = list(rng.choice(VOCAB, size=rng.integers(0, 4), replace=False))
            meta[nid] = tuple(str(rng.choice(m)) or d for m, d in zip(META, DEFAULT))
        st.set_routes(ids0, [blocks[i] for i in ids0], [lex[i] for i in ids0],
                      [meta[i] for i in ids0])
        for step in range(30):
            if step % 5 == 4:
                for nid in rng.choice(sorted(blocks), size=15, replace=False):
                    nid = int(nid)
                    op = rng.integers(0, 3)
                    if op == 0:
                        blocks[nid] = rng.standard_normal(
                            (kv, int(rng.integers(0, 40)), hd)).astype(np.float32)
                        lex[nid] = list(rng.choice(VOCAB, size=rng.integers(0, 3), replace=False))
                        st.set_route(nid, blocks[nid], lex[nid])
                    elif op == 1:
                        vals = tuple(str(rng.choice(m)) for m in META)
                        st.set_route_metadata(nid, *vals)
                        meta[nid] = tuple(v if v else o for v, o in zip(vals, meta[nid]))
                    else:
                        st.clear_route(nid)
                        del blocks[nid], lex[nid], meta[nid]
            ids = sorted(blocks)
            lens = np.asarray([blocks[i].shape[1] for i in ids], dtype=np.uint64)
            offs = np.zeros(len(ids) + 1, dtype=np.uint64)
            offs[1:] = np.cumsum(lens)
            keys = np.concatenate([blocks[i].reshape(-1) for i in ids])
            Qt = int(rng.integers(1, 6))
            q = rng.standard_normal((H, Qt, hd)).astype(np.float32)
            qlex = list(rng.choice(VOCAB, size=rng.integers(0, 5), replace=True))
            filters = tuple([str(v) for v in rng.choice(m, size=rng.integers(0, 3), replace=False)
                             if v] if rng.random() < 0.5 else [] for m in META)
            k = int(rng.integers(1, 16))
            want_ids, want_sc = oracle.store_route_gqa(
                keys, offs, kv, hd, ids, [lex[i] for i in ids], [meta[i] for i in ids], q, qlex,
                filters, k)
            got_ids, got_sc = st.route_scored(q, qlex, k, kinds=filters[0], scopes=filters[1],
                                              durabilities=filters[2], mutabilities=filters[3])
            assert got_ids == want_ids, (step, qlex, filters, k)
            np.testing.assert_array_equal(np.asarray(got_sc, np.float32).view(np.uint32),
                                          want_sc.view(np.uint32))
            assert st.route_gqa(q, "\n".join(qlex), *["\n".join(f) for f in filters],
                                topk=k) == want_ids


def test_device_store_refuses_what_it_does_not_serve(hip_lib):
    from graftrepository_amd import _lib
    from graftrepository_amd.store_route import DeviceGqaRouteStore

    lib = _lib.load()
    with DeviceRouteStore(8, capacity=64) as st:
        with pytest.raises(RuntimeError):
            st.set_route(1, np.zeros(7, np.float32))          # wrong length
        keys = np.zeros((2, 7), np.float32)
        rc = lib.grm_store_set_route_multi(st._h, 3, keys.ctypes.data, 2, 7, b"")
        assert rc != 0 and b"dim" in lib.grm_store_last_error(st._h)   # rows of another length
        offs = np.asarray([0, 8, 4], np.uint64)
        rc = lib.grm_store_set_route_list(st._h, 3, keys.ctypes.data, 4, offs.ctypes.data, 2, b"")
        assert rc != 0                                          # offsets out of order
        st.set_route(1, np.ones(8, np.float32), "a")
        with pytest.raises(RuntimeError):
            st.route_scored(np.ones(8, np.float32), topk=17)   # above the device list
        st.clear_route(99)                                     # no entry: nothing to clear
        assert len(st) == 1
    with DeviceGqaRouteStore(2, 8, capacity_nodes=8, capacity_tokens=64) as st:
        with pytest.raises(RuntimeError):
            st.set_route(1, np.zeros(17, np.float32))         # not whole [kv][L][hd] blocks
        q = np.zeros((3, 1, 8), np.float32)
        with pytest.raises(RuntimeError):
            st.route_gqa(q, topk=2)                             # heads not a multiple of kv


def _multi_case(rng, make_key):
    k = int(rng.integers(0, 4))
    keys = [make_key() for _ in range(k)]
    if k > 1 and rng.random() < 0.3 and keys[0].size:
        keys[0] = keys[0].copy()
        keys[0].reshape(-1)[0] = np.nan
    return keys


@pytest.mark.parametrize("dialect", ["mla", "gqa"])
def test_device_store_multi_key_entries_match_the_law(hip_lib, dialect):
    # entries of several keys score their best finite key
    # (exact_mla_entry_score cpp/grm_runtime.cpp:3518-3545; max_gqa_raw_score
    # :3031-3051); law pinned against the reference store in
    # test_store_route.py
    from graftrepository_amd.store_route import DeviceGqaRouteStore

    rng = np.random.default_rng(57 if dialect == "mla" else 58)
    if dialect == "mla":
        n, dim = 1500, 48
        make = lambda: rng.standard_normal(dim).astype(np.float32)
        st = DeviceRouteStore(dim, capacity=2048)
    else:
        n, kv, hd, H = 300, 2, 64, 8
        make = lambda: rng.standard_normal((kv, int(rng.integers(0, 30)), hd)).astype(np.float32)
        st = DeviceGqaRouteStore(kv, hd, capacity_nodes=512, capacity_tokens=30_000)
    entries, lex, meta = {}, {}, {}

    def put(nid, keys):
        entries[nid] = keys
        lex[nid] = list(rng.choice(VOCAB, size=rng.integers(0, 4), replace=False))
        if len(keys) == 1 and rng.random() < 0.5:
            st.set_route(nid, keys[0], lex[nid])
        elif dialect == "mla" and len(keys) > 0 and rng.random() < 0.5:
            st.set_route_multi(nid, np.stack(keys), lex[nid])
        else:
            st.set_route_list(nid, keys, lex[nid])
        meta.setdefault(nid, DEFAULT)

    with st:
        for i in range(n):
            put(2000 + i, _multi_case(rng, make) if i % 3 == 0 else [make()])
        entries[2009] = [entries[2003][0].copy()] if entries[2003] else [make()]
        st.set_route(2009, entries[2009][0], lex[2009])          # a tie across entries
        for step in range(24):
            if step % 4 == 3:
                for nid in rng.choice(sorted(entries), size=12, replace=False):
                    nid = int(nid)
                    op = rng.integers(0, 3)
                    if op == 0:
                        put(nid, _multi_case(rng, make) if rng.random() < 0.5 else [make()])
                    elif op == 1:
                        vals = tuple(str(rng.choice(m)) for m in META)
                        st.set_route_metadata(nid, *vals)
                        meta[nid] = tuple(v if v else o for v, o in zip(vals, meta[nid]))
                    else:
                        st.clear_route(nid)
                        del entries[nid], lex[nid], meta[nid]
            ids = sorted(entries)
            owners = [j for j, nid in enumerate(ids) for _ in entries[nid]]
            flat = [key for nid in ids for key in entries[nid]]
            qlex = list(rng.choice(VOCAB, size=rng.integers(0, 5), replace=True))
            filters = tuple([str(v) for v in rng.choice(m, size=rng.integers(0, 3), replace=False)
                             if v] if rng.random() < 0.5 else [] for m in META)
            k = int(rng.integers(1, 17))
            lexs, metas = [lex[i] for i in ids], [meta[i] for i in ids]
            if dialect == "mla":
                q = rng.standard_normal(dim).astype(np.float32)
                want_ids, want_sc = oracle.store_route(np.stack(flat), ids, lexs, metas, q, qlex,
                                                       filters, k, owners=owners)
            else:
                lens = np.asarray([b.shape[1] for b in flat], dtype=np.uint64)
                offs = np.zeros(len(flat) + 1, dtype=np.uint64)
                offs[1:] = np.cumsum(lens)
                keys = np.concatenate([b.reshape(-1) for b in flat])
                q = rng.standard_normal((H, int(rng.integers(1, 4)), hd)).astype(np.float32)
                want_ids, want_sc = oracle.store_route_gqa(keys, offs, kv, hd, ids, lexs, metas,
                                                           q, qlex, filters, k, owners=owners)
            got_ids, got_sc = st.route_scored(q, qlex, k, kinds=filters[0], scopes=filters[1],
                                              durabilities=filters[2], mutabilities=filters[3])
            assert got_ids == want_ids, (step, qlex, filters, k)
            np.testing.assert_array_equal(np.asarray(got_sc, np.float32).view(np.uint32),
                                          want_sc.view(np.uint32))


def test_device_gqa_store_topk16_with_lexical_keys(hip_lib):
    # k = 16 is the bank's list cap, so a lexical route fetches 16, not
    # k + 1; the guard then rests on fl(pred(r_16) / norm) (csrc/store.hip).
    # Raw ties (duplicate blocks) straddle the 16th place.  Ids and scores
    # must equal the law.
    from graftrepository_amd.store_route import DeviceGqaRouteStore

    rng = np.random.default_rng(57)
    n, kv, hd, H = 300, 2, 32, 8
    blocks = {700 + i: rng.standard_normal((kv, int(rng.integers(1, 30)), hd)).astype(np.float32)
              for i in range(n)}
    for a in range(700, 760, 3):
        blocks[a + 1] = blocks[a].copy()
    lex = {nid: (list(rng.choice(VOCAB, size=2, replace=False)) if rng.random() < 0.1 else [])
           for nid in blocks}
    meta = {nid: DEFAULT for nid in blocks}
    ids = sorted(blocks)
    lens = np.asarray([blocks[i].shape[1] for i in ids], dtype=np.uint64)
    offs = np.zeros(len(ids) + 1, dtype=np.uint64)
    offs[1:] = np.cumsum(lens)
    keys = np.concatenate([blocks[i].reshape(-1) for i in ids])
    with DeviceGqaRouteStore(kv, hd, capacity_nodes=400, capacity_tokens=20_000) as st:
        st.set_routes(ids, [blocks[i] for i in ids], [lex[i] for i in ids],
                      [meta[i] for i in ids])
        for step in range(25):
            q = rng.standard_normal((H, int(rng.integers(1, 3)), hd)).astype(np.float32)
            qlex = list(rng.choice(VOCAB, size=int(rng.integers(1, 4)), replace=True))
            want_ids, want_sc = oracle.store_route_gqa(
                keys, offs, kv, hd, ids, [lex[i] for i in ids], [meta[i] for i in ids], q, qlex,
                ((), (), (), ()), 16)
            got_ids, got_sc = st.route_scored(q, qlex, 16)
            assert got_ids == want_ids, step
            np.testing.assert_array_equal(np.asarray(got_sc, np.float32).view(np.uint32),
                                          want_sc.view(np.uint32))


def test_device_store_put_that_cannot_fit_keeps_the_old_entry(hip_lib):
    # A set_route / set_route_multi whose new keys cannot fit once the old
    # ones are gone fails before touching the entry: it stays routable with
    # its old key.
    from graftrepository_amd.store_route import DeviceGqaRouteStore

    rng = np.random.default_rng(59)
    # GQA: 4 nodes of 8 tokens in a bank of 4 nodes and 32 tokens (the bank
    # adds 7 tokens of alignment room per node: 60 in all)
    kv, hd, H = 2, 16, 4
    with DeviceGqaRouteStore(kv, hd, capacity_nodes=4, capacity_tokens=32) as st:
        blocks = {i: rng.standard_normal((kv, 8, hd)).astype(np.float32) for i in range(4)}
        for i, b in blocks.items():
            st.set_route(i, b)
        q = blocks[0][:, :1, :].repeat(2, axis=0).copy()   # matches node 0 best
        before = st.route_scored(q, (), 4)
        assert before[0][0] == 0
        with pytest.raises(RuntimeError, match="unchanged"):
            st.set_route(0, rng.standard_normal((kv, 40, hd)).astype(np.float32))
        assert st.route_scored(q, (), 4) == before
        with pytest.raises(RuntimeError):
            st.set_route(9, blocks[1])                         # a fifth node
        assert st.route_scored(q, (), 4) == before and len(st) == 4
        st.set_route(0, rng.standard_normal((kv, 32, hd)).astype(np.float32))  # fits
        assert len(st) == 4 and st.route_scored(q, (), 4) != before
    # MLA: 64 slots full; a new entry fails, a replacement fits; a multi-key
    # entry with more keys than its bank holds fails and keeps the old key
    dim = 12
    with DeviceRouteStore(dim, capacity=64) as st:
        rows = {i: rng.standard_normal(dim).astype(np.float32) for i in range(64)}
        for i, r in rows.items():
            st.set_route(i, r)
        q = rows[5].copy()
        before = st.route_scored(q, (), 3)
        with pytest.raises(RuntimeError, match="unchanged"):
            st.set_route(100, rows[1])
        assert st.route_scored(q, (), 3) == before and len(st) == 64
        with pytest.raises(RuntimeError, match="unchanged"):
            st.set_route_multi(5, rng.standard_normal((65, dim)).astype(np.float32))
        assert st.route_scored(q, (), 3) == before
        st.set_route(5, -rows[5])                              # a replacement fits
        assert st.route_scored(q, (), 3)[0][0] != 5
