"""The store's MLA route on the device: lexical bonus and route filters.

Counterpart of the CPU store's route calls for MLA stores:

* ``grm_store_set_route`` / ``grm_store_clear_route``
  (cpp/grm_runtime_c.h:381-401);
* ``grm_store_set_route_metadata`` (:176-181);
* ``grm_store_route`` / ``grm_store_route_filtered`` (:402-424).

Their law is ``route_mla_arena`` (cpp/grm_runtime.cpp:4299-4361):

* an entry takes part if it passes the route filters (:3074-3104);
* its exact MLA score must be finite (:3518-3545);
* its route score is that score plus the lexical bonus, both in float:
  hits / |query lexical keys| (:3133-3170);
* a non-finite sum drops the entry;
* entries sort by (score desc, node id asc).

How the device answers it:

* The bank scores every node with the filters applied.  A filtered-out
  node gets a NaN norm for that route, so it never ranks.
* The bonus is never negative, so fl(score + bonus) >= score.  A node
  without lexical hits that ends in the top k therefore already lies in
  the filtered device top k of plain scores.  Were it outside, k nodes
  would beat it on score and so on score + bonus.
* The answer therefore lies among that device top k and the nodes with
  lexical hits.  The latter are found through a host index of lexical
  keys and scored exactly on the device (``grm_mla_hip_score_nodes``),
  then the union is ranked by the law.

Filter values the reference knows (:2797-2827) are bits on each node.  A
category filtered by any other value compares the node's own string, as
the reference does (:3053-3057, 3074-3086).  That is served by a per-query
match bit, set on the matching nodes for the one route.

Multi-row entries (``grm_store_set_route_multi`` / ``_list``) are not
served; the reference's device route declines them too
(core/graft_arena.py:1128-1131).
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from .node_bank import MlaNodeBank, _ptr

NO_ID = np.iinfo(np.uint64).max

# known route filter values and their bits (cpp/grm_runtime.cpp:2788-2827)
_SHIFTS = {"kind": 0, "scope": 16, "durability": 32, "mutability": 48}
_KNOWN = {
    "kind": ("turn", "doc", "digest", "era", "fact", "task_state", "recall", "cull_span"),
    "scope": ("conversation", "project", "user", "task", "global", "session"),
    "durability": ("volatile", "session", "project", "permanent"),
    "mutability": ("ephemeral", "stable", "mutable", "immutable"),
}
_MATCH_BIT = 15  # unused by every known value: the per-query string-match bit
_CATS = ("kind", "scope", "durability", "mutability")
# a new route entry's metadata (cpp/grm_runtime.hpp:483-494)
_DEFAULT_META = ("turn", "conversation", "session", "ephemeral")


def split_keys(keys) -> list[str]:
    """Lexical keys or filter values: a list of strings, or one
    '\\n'-joined string split on newlines with empty items dropped
    (cpp/grm_runtime.cpp:5196-5209)."""
    if keys is None:
        return []
    if isinstance(keys, (bytes, str)):
        text = keys.decode("utf-8") if isinstance(keys, bytes) else keys
        return [s for s in text.split("\n") if s]
    return [str(s) for s in keys if str(s)]


def known_bit(category: str, value: str) -> int:
    values = _KNOWN[category]
    return (1 << (_SHIFTS[category] + values.index(value))) if value in values else 0


def filter_bits(kind="", scope="", durability="", mutability="") -> int:
    """A node's route filter bits (cpp/grm_runtime.cpp:2829-2838)."""
    vals = dict(kind=kind, scope=scope, durability=durability, mutability=mutability)
    out = 0
    for c in _CATS:
        out |= known_bit(c, vals[c])
    return out


class DeviceRouteStore:
    """MLA store route served by a device bank.  Node ids are the store's.
    ``route`` / ``route_filtered`` return node ids like the reference ABI;
    ``route_scored`` also returns the route scores."""

    def __init__(self, dim: int, *, dtype: str = "f32", capacity: int = 1024):
        self.dim = int(dim)
        self.bank = MlaNodeBank(None, dtype=dtype, dim=self.dim, capacity=max(64, int(capacity)))
        self._lib = _lib.load()
        self._lex: dict[int, list[str]] = {}           # node -> its lexical keys
        self._index: dict[str, set[int]] = {}          # lexical key -> nodes
        self._meta: dict[int, tuple] = {}              # node -> (kind, scope, dur, mut)
        self._bits: dict[int, int] = {}                # node -> filter bits on the device

    def close(self) -> None:
        if self.bank is not None:
            self.bank.close()
            self.bank = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ------------------------------------------------------------ mutation
    def _grow(self, extra: int) -> None:
        info = self.bank.info()
        if info["live"] + extra > info["capacity"]:
            # the bank keeps no host copy of its rows; its capacity is fixed
            raise RuntimeError(f"device route store is full (capacity {info['capacity']})")

    def set_route(self, node_id: int, route_key, lexical_keys=()) -> None:
        nid = int(node_id)
        key = np.ascontiguousarray(route_key, dtype=np.float32).reshape(1, -1)
        if key.shape[1] != self.dim:
            raise ValueError(f"route key has {key.shape[1]} values, the store {self.dim}")
        if nid in self._lex:
            self.bank.evict([nid])
            self._unindex(nid)
        else:
            self._grow(1)
        self.bank.append(key, [nid])
        lex = split_keys(lexical_keys)
        self._lex[nid] = lex
        for s in set(lex):
            self._index.setdefault(s, set()).add(nid)
        # a new entry starts from the defaults; a replaced one keeps its
        # metadata (cpp/grm_runtime.cpp:2877-2902)
        meta = self._meta.setdefault(nid, _DEFAULT_META)
        bits = filter_bits(*meta)
        self._bits[nid] = bits
        self._set_bits([nid], [bits])

    def set_routes(self, node_ids, route_keys, lexical_keys=None, metadata=None) -> None:
        """Many new nodes at once: one append and one filter-bits upload.
        lexical_keys[i] / metadata[i] (kind, scope, durability, mutability;
        empty values keep the defaults) may be omitted."""
        ids = np.ascontiguousarray(node_ids, dtype=np.uint64).reshape(-1)
        keys = np.ascontiguousarray(route_keys, dtype=np.float32).reshape(ids.size, -1)
        if keys.shape[1] != self.dim:
            raise ValueError("route keys do not match the store dim")
        if any(int(n) in self._lex for n in ids):
            raise ValueError("set_routes takes new node ids only")
        self._grow(ids.size)
        self.bank.append(keys, ids)
        bits = np.empty(ids.size, dtype=np.uint64)
        for j, n in enumerate(ids.tolist()):
            lex = split_keys(lexical_keys[j]) if lexical_keys is not None else []
            self._lex[n] = lex
            for s_ in set(lex):
                self._index.setdefault(s_, set()).add(n)
            m = _DEFAULT_META
            if metadata is not None:
                m = tuple(str(v) if v else o for v, o in zip(metadata[j], _DEFAULT_META))
            self._meta[n] = m
            b = filter_bits(*m)
            self._bits[n] = b
            bits[j] = b
        self._set_bits(ids, bits)

    def set_route_metadata(self, node_id: int, kind="", scope="", durability="",
                           mutability="") -> None:
        """Non-empty values replace the entry's; a node without a route
        entry is left alone (cpp/grm_runtime.cpp:2922-2946)."""
        nid = int(node_id)
        if nid not in self._lex:
            return
        new = (str(kind), str(scope), str(durability), str(mutability))
        self._meta[nid] = tuple(n if n else o for n, o in zip(new, self._meta[nid]))
        bits = filter_bits(*self._meta[nid])
        self._bits[nid] = bits
        self._set_bits([nid], [bits])

    def clear_route(self, node_id: int) -> None:
        nid = int(node_id)
        if nid not in self._lex:
            raise KeyError(nid)
        self.bank.evict([nid])
        self._unindex(nid)
        del self._lex[nid]
        self._bits.pop(nid, None)
        self._meta.pop(nid, None)

    def _unindex(self, nid: int) -> None:
        for s in set(self._lex.get(nid, ())):
            nodes = self._index.get(s)
            if nodes is not None:
                nodes.discard(nid)
                if not nodes:
                    del self._index[s]

    def _set_bits(self, nids, bits) -> None:
        ids = np.ascontiguousarray(nids, dtype=np.uint64)
        b = np.ascontiguousarray(bits, dtype=np.uint64)
        _lib.check(self._lib.grm_mla_hip_set_filter_bits(self.bank._h, _ptr(ids), _ptr(b),
                                                         ids.size), "set filter bits")

    # --------------------------------------------------------------- route
    def _allowed_host(self, nid: int, masks: dict, strings: dict) -> bool:
        meta = self._meta.get(nid, _DEFAULT_META)
        bits = self._bits.get(nid, 0)
        for ci, c in enumerate(_CATS):
            if c in masks and not (bits & masks[c]):
                return False
            if c in strings and meta[ci] not in strings[c]:
                return False
        return True

    def route_scored(self, query, lexical_keys=(), topk: int = 3, *, kinds=(), scopes=(),
                     durabilities=(), mutabilities=()):
        """(node ids, route scores) of the store's route law, best first."""
        if not 1 <= int(topk) <= 16:
            raise ValueError("topk must be in [1, 16]")
        q = np.ascontiguousarray(query, dtype=np.float32).reshape(-1)
        if q.size != self.dim:
            raise ValueError("query dim does not match the store")
        k = int(topk)
        lex = split_keys(lexical_keys)
        filters = dict(zip(_CATS, (split_keys(kinds), split_keys(scopes),
                                   split_keys(durabilities), split_keys(mutabilities))))
        masks, strings = {}, {}
        for c, vals in filters.items():
            if not vals:
                continue
            bits = [known_bit(c, v) for v in vals]
            if all(bits):
                masks[c] = int(np.bitwise_or.reduce(np.asarray(bits, dtype=np.uint64)))
            else:
                strings[c] = set(vals)
        live = len(self._lex)
        if live == 0:
            return [], []
        # categories filtered by strings: a match bit on the matching nodes
        temp = {}
        for c, vals in strings.items():
            ci = _CATS.index(c)
            bit = 1 << (_SHIFTS[c] + _MATCH_BIT)
            for nid in self._lex:
                if self._meta.get(nid, _DEFAULT_META)[ci] in vals:
                    temp[nid] = temp.get(nid, self._bits.get(nid, 0)) | bit
            masks[c] = bit
        if temp:
            self._set_bits(list(temp), list(temp.values()))
        try:
            fmask = 0
            cats = 0
            for ci, c in enumerate(_CATS):
                if c in masks:
                    fmask |= masks[c]
                    cats |= 1 << ci
            kk = min(k, live)
            ids = np.empty((1, kk), dtype=np.uint64)
            sc = np.empty((1, kk), dtype=np.float32)
            # no device time asked for: the library waits on completion flags
            _lib.check(self._lib.grm_mla_hip_route_filtered(
                self.bank._h, _ptr(q), 0, 0, kk, ctypes.c_uint64(fmask), ctypes.c_uint32(cats),
                _ptr(ids), _ptr(sc), None), "store route")
        finally:
            if temp:
                self._set_bits(list(temp), [self._bits.get(n, 0) for n in temp])
        cand = {int(n): float(s) for n, s in zip(ids[0], sc[0])
                if n != NO_ID and np.isfinite(s)}
        bonus = {}
        if lex:
            hits: dict[int, int] = {}
            for s in lex:                       # each query key counts once per entry hit
                for nid in self._index.get(s, ()):
                    hits[nid] = hits.get(nid, 0) + 1
            den = np.float32(len(lex))
            for nid, h in hits.items():
                if self._allowed_host(nid, {c: m for c, m in masks.items() if c not in strings},
                                      strings):
                    bonus[nid] = np.float32(h) / den
            need = [n for n in bonus if n not in cand]
            if need:
                ids2 = np.asarray(need, dtype=np.uint64)
                out = np.empty(ids2.size, dtype=np.float32)
                _lib.check(self._lib.grm_mla_hip_score_nodes(
                    self.bank._h, _ptr(q), 0, _ptr(ids2), ids2.size, _ptr(out)), "score nodes")
                for n, s in zip(need, out):
                    if np.isfinite(s):
                        cand[int(n)] = float(s)
        scored = []
        for nid, base in cand.items():
            total = np.float32(base) + bonus.get(nid, np.float32(0.0))
            if np.isfinite(total):
                scored.append((-float(total), nid, np.float32(total)))
        scored.sort()
        top = scored[:k]
        return [n for _, n, _ in top], [float(s) for _, _, s in top]

    def route(self, query, lexical_keys=(), topk: int = 3) -> list[int]:
        """``grm_store_route``: node ids, best first."""
        return self.route_scored(query, lexical_keys, topk)[0]

    def route_filtered(self, query, lexical_keys=(), kinds=(), scopes=(), durabilities=(),
                       mutabilities=(), topk: int = 3) -> list[int]:
        """``grm_store_route_filtered``: node ids, best first."""
        return self.route_scored(query, lexical_keys, topk, kinds=kinds, scopes=scopes,
                                 durabilities=durabilities, mutabilities=mutabilities)[0]


__all__ = ["DeviceRouteStore", "filter_bits", "known_bit", "split_keys"]
