"""The store route law (lexical bonus and route filters) on the CPU: the
oracle's restatement pinned against the reference store itself.

The reference store is ``cpp/grm_runtime.cpp``, built into oracle/_ref.
The cases are random stores with a small shared lexical vocabulary
(collisions and repeated query keys), duplicate rows (score ties), route
metadata drawn from known values, unknown values and empty values, and
filters of known and unknown values.  Law: route_mla_arena
(cpp/grm_runtime.cpp:4299-4361).
"""

import numpy as np
import pytest

import oracle
from oracle import ref
from graftrepository_amd import store_route as sr

pytestmark = pytest.mark.skipif(not ref.available(), reason="reference CPU store not built")

VOCAB = ["alpha", "beta", "gamma", "delta", "eps", "zeta", "eta", "theta", "iota", "kappa"]
META = [
    ["turn", "doc", "fact", "recall", "weird-kind", ""],
    ["conversation", "project", "global", "elsewhere", ""],
    ["volatile", "permanent", "session", ""],
    ["stable", "mutable", "odd", ""],
]


def random_store(rng, n, dim):
    rows = rng.standard_normal((n, dim)).astype(np.float32)
    rows[5] = rows[4]                              # exact ties
    rows[9] = rows[4]
    lexical = [list(rng.choice(VOCAB, size=rng.integers(0, 4), replace=False)) for _ in range(n)]
    meta = [tuple(str(rng.choice(m)) for m in META) for _ in range(n)]
    return rows, lexical, meta


def random_query(rng, rows, dim):
    q = rng.standard_normal(dim).astype(np.float32)
    if rng.random() < 0.3:
        q = rows[4].copy()
    qlex = list(rng.choice(VOCAB, size=rng.integers(0, 5), replace=True))
    filters = tuple(list(rng.choice(m, size=rng.integers(0, 3), replace=False))
                    if rng.random() < 0.5 else [] for m in META)
    return q, qlex, tuple([v for v in f if v] for f in filters)


def test_oracle_store_law_matches_the_reference_store():
    rng = np.random.default_rng(41)
    n, dim = 120, 12
    rows, lexical, meta = random_store(rng, n, dim)
    for case in range(60):
        q, qlex, filters = random_query(rng, rows, dim)
        k = int(rng.integers(1, 17))
        want = ref.store_route(rows, lexical, meta, q, qlex, filters, k)
        got, _ = oracle.store_route(rows, np.arange(n), lexical, meta, q, qlex, filters, k)
        assert got == want, (case, qlex, filters, k)


def test_lexical_bonus_reorders_and_filters_bind():
    rng = np.random.default_rng(42)
    rows, lexical, meta = random_store(rng, 80, 8)
    q = rng.standard_normal(8).astype(np.float32)
    plain, _ = oracle.store_route(rows, np.arange(80), lexical, meta, q, (), ((), (), (), ()), 5)
    boosted, _ = oracle.store_route(rows, np.arange(80), lexical, meta, q,
                                    ["alpha", "beta"], ((), (), (), ()), 5)
    assert plain != boosted
    assert boosted == ref.store_route(rows, lexical, meta, q, ["alpha", "beta"],
                                      ((), (), (), ()), 5)
    only_docs, _ = oracle.store_route(rows, np.arange(80), lexical, meta, q, (),
                                      (["doc"], (), (), ()), 16)
    assert only_docs and all(meta[i][0] == "doc" for i in only_docs)


def test_split_and_bits_follow_the_reference():
    assert sr.split_keys("a\n\nb\n") == ["a", "b"]
    assert sr.split_keys(b"x\ny") == ["x", "y"]
    assert sr.split_keys(["a", "", "b"]) == ["a", "b"]
    assert sr.filter_bits("doc", "project", "permanent", "stable") == (
        (1 << 1) | (1 << 17) | (1 << 35) | (1 << 49))
    assert sr.filter_bits("weird", "", "", "") == 0


def random_gqa_store(rng, n, kv, hd):
    lens = rng.integers(0, 20, size=n)
    blocks = [rng.standard_normal((kv, int(L), hd)).astype(np.float32) for L in lens]
    blocks[5] = blocks[4].copy()                   # exact ties
    blocks[9] = blocks[4].copy()
    lexical = [list(rng.choice(VOCAB, size=rng.integers(0, 4), replace=False)) for _ in range(n)]
    meta = [tuple(str(rng.choice(m)) for m in META) for _ in range(n)]
    return blocks, lexical, meta


def test_oracle_gqa_store_law_matches_the_reference_store():
    rng = np.random.default_rng(43)
    n, kv, hd, H = 80, 2, 8, 4
    blocks, lexical, meta = random_gqa_store(rng, n, kv, hd)
    lens = np.asarray([b.shape[1] for b in blocks], dtype=np.uint64)
    offs = np.zeros(n + 1, dtype=np.uint64)
    offs[1:] = np.cumsum(lens)
    keys = np.concatenate([b.reshape(-1) for b in blocks])
    for case in range(60):
        Qt = int(rng.integers(1, 4))
        q = rng.standard_normal((H, Qt, hd)).astype(np.float32)
        if rng.random() < 0.3 and blocks[4].shape[1] > 0:
            q[:, 0, :] = np.repeat(blocks[4][:, 0, :], H // kv, axis=0)
        qlex = list(rng.choice(VOCAB, size=rng.integers(0, 5), replace=True))
        filters = tuple([v for v in (list(rng.choice(m, size=rng.integers(0, 3), replace=False))
                                     if rng.random() < 0.5 else []) if v] for m in META)
        k = int(rng.integers(1, 17))
        want = ref.store_route_gqa(blocks, lexical, meta, q, kv, qlex, filters, k)
        got, _ = oracle.store_route_gqa(keys, offs, kv, hd, np.arange(n), lexical, meta, q,
                                        qlex, filters, k)
        assert got == want, (case, qlex, filters, k)


def multi_entries(rng, n, make_key, max_keys=3):
    """Entries of 0..max_keys keys; a few keys not finite."""
    entries, owners, flat = [], [], []
    for i in range(n):
        k = int(rng.integers(0, max_keys + 1)) if i % 4 == 0 else 1
        keys = [make_key() for _ in range(k)]
        if k > 1 and i % 8 == 0 and keys[0].size:
            keys[0] = keys[0].copy()
            keys[0].reshape(-1)[0] = np.nan                 # one key not finite
        entries.append(keys)
        for key in keys:
            owners.append(i)
            flat.append(key)
    return entries, owners, flat


def test_oracle_multi_row_mla_law_matches_the_reference_store():
    # multi-row entries score their best finite row (exact_mla_entry_score,
    # cpp/grm_runtime.cpp:3518-3545); an entry with no finite row drops out
    rng = np.random.default_rng(44)
    n, dim = 90, 10
    entries, owners, flat = multi_entries(rng, n, lambda: rng.standard_normal(dim).astype(np.float32))
    entries[7] = [entries[3][0].copy()] if entries[3] else entries[7]   # a tie across entries
    owners = [i for i, e in enumerate(entries) for _ in e]
    flat = [k for e in entries for k in e]
    rows = np.stack(flat)
    _, lexical, meta = random_store(rng, n, dim)
    for case in range(40):
        q, qlex, filters = random_query(rng, rows, dim)
        k = int(rng.integers(1, 17))
        want = ref.store_route(entries, lexical, meta, q, qlex, filters, k)
        got, _ = oracle.store_route(rows, np.arange(n), lexical, meta, q, qlex, filters, k,
                                    owners=owners)
        assert got == want, (case, qlex, filters, k)


def test_oracle_multi_key_gqa_law_matches_the_reference_store():
    # multi-key entries score their best finite key (max_gqa_raw_score,
    # cpp/grm_runtime.cpp:3031-3051)
    rng = np.random.default_rng(45)
    n, kv, hd, H = 60, 2, 8, 4
    entries, owners, flat = multi_entries(
        rng, n, lambda: rng.standard_normal((kv, int(rng.integers(0, 12)), hd)).astype(np.float32))
    lens = np.asarray([b.shape[1] for b in flat], dtype=np.uint64)
    offs = np.zeros(len(flat) + 1, dtype=np.uint64)
    offs[1:] = np.cumsum(lens)
    keys = np.concatenate([b.reshape(-1) for b in flat])
    _, lexical, meta = random_gqa_store(rng, n, kv, hd)
    for case in range(40):
        Qt = int(rng.integers(1, 3))
        q = rng.standard_normal((H, Qt, hd)).astype(np.float32)
        qlex = list(rng.choice(VOCAB, size=rng.integers(0, 5), replace=True))
        filters = tuple([v for v in (list(rng.choice(m, size=rng.integers(0, 3), replace=False))
                                     if rng.random() < 0.5 else []) if v] for m in META)
        k = int(rng.integers(1, 17))
        want = ref.store_route_gqa(entries, lexical, meta, q, kv, qlex, filters, k)
        got, _ = oracle.store_route_gqa(keys, offs, kv, hd, np.arange(n), lexical, meta, q,
                                        qlex, filters, k, owners=owners)
        assert got == want, (case, qlex, filters, k)
