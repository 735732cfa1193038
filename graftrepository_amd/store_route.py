"""The store's route calls on the device: lexical bonus and route filters.

Python face of the library's device store (``csrc/store.hip``), which serves
the CPU store's route calls with their names and argument lists
(cpp/grm_runtime_c.h:176-181, 381-436):

* ``grm_store_set_route`` / ``_set_route_multi`` / ``_set_route_list`` /
  ``grm_store_clear_route`` / ``grm_store_set_route_metadata``;
* ``grm_store_route`` / ``grm_store_route_filtered`` (MLA stores, law
  ``route_mla_arena``, cpp/grm_runtime.cpp:4299-4361);
* ``grm_store_route_gqa`` (GQA stores, law ``route_gqa_raw``, :4498-4881).

The laws, and how the device answers them (the filtered bank top k plus
every entry with lexical hits, scored exactly on the device, ranked by the
law), are described in ``csrc/store.hip``.  ``DeviceRouteStore`` (MLA) and
``DeviceGqaRouteStore`` hold a handle; ``route_scored`` also returns the
fp32 route scores the law ranks by.

Entries with several route keys (``set_route_multi`` / ``set_route_list``)
score their best finite key, as the reference's store does
(cpp/grm_runtime.cpp:3518-3545, 3031-3051); the library scores their keys
exactly on every route.
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from .node_bank import _ptr

NO_ID = np.iinfo(np.uint64).max

# known route filter values and their bits (cpp/grm_runtime.cpp:2788-2827)
_SHIFTS = {"kind": 0, "scope": 16, "durability": 32, "mutability": 48}
_KNOWN = {
    "kind": ("turn", "doc", "digest", "era", "fact", "task_state", "recall", "cull_span"),
    "scope": ("conversation", "project", "user", "task", "global", "session"),
    "durability": ("volatile", "session", "project", "permanent"),
    "mutability": ("ephemeral", "stable", "mutable", "immutable"),
}
_CATS = ("kind", "scope", "durability", "mutability")


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


def _blob(keys) -> bytes:
    return "\n".join(split_keys(keys)).encode("utf-8")


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


class _Store:
    """One device store handle (route entries of one dialect)."""

    def __init__(self, handle: ctypes.c_void_p):
        self._lib = _lib.load()
        self._h = handle

    def close(self) -> None:
        if self._h is not None and self._h.value:
            self._lib.grm_hip_store_destroy(self._h)
        self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def _check(self, rc: int, what: str) -> None:
        if rc != 0:
            msg = self._lib.grm_store_last_error(self._h)
            detail = msg.decode("utf-8", "replace") if msg else ""
            raise RuntimeError(f"{what} failed with code {rc}" + (f": {detail}" if detail else ""))

    def _need_open(self):
        if self._h is None or not self._h.value:
            raise RuntimeError("store is closed")

    def __len__(self) -> int:
        self._need_open()
        out = np.zeros(4, dtype=np.uint64)
        self._check(self._lib.grm_hip_store_info(self._h, _ptr(out)), "store info")
        return int(out[1])

    # ------------------------------------------------------------ mutation
    def set_route(self, node_id: int, route_key, lexical_keys=()) -> None:
        self._need_open()
        key = np.ascontiguousarray(route_key, dtype=np.float32).reshape(-1)
        self._check(self._lib.grm_store_set_route(self._h, int(node_id), _ptr(key), key.size,
                                                  _blob(lexical_keys)), "set_route")

    def set_route_list(self, node_id: int, route_keys, lexical_keys=()) -> None:
        """``grm_store_set_route_list``: the entry's keys (any number, each
        a whole route key; MLA rows of the store's dim, GQA [kv][L][hd]
        blocks).  It scores the best of them."""
        self._need_open()
        flat = [np.ascontiguousarray(k, dtype=np.float32).reshape(-1) for k in route_keys]
        values = np.concatenate(flat) if flat else np.zeros(0, np.float32)
        offs = np.zeros(len(flat) + 1, dtype=np.uint64)
        offs[1:] = np.cumsum([f.size for f in flat])
        self._check(self._lib.grm_store_set_route_list(
            self._h, int(node_id), _ptr(values), values.size, _ptr(offs), len(flat),
            _blob(lexical_keys)), "set_route_list")

    def set_route_multi(self, node_id: int, route_keys, lexical_keys=()) -> None:
        """``grm_store_set_route_multi``: keys of one length, [keys, len]."""
        self._need_open()
        k = np.ascontiguousarray(route_keys, dtype=np.float32)
        k = k.reshape(k.shape[0], -1) if k.ndim >= 1 and k.size else k.reshape(0, 0)
        self._check(self._lib.grm_store_set_route_multi(
            self._h, int(node_id), _ptr(k), k.shape[0], k.shape[1] if k.ndim == 2 else 0,
            _blob(lexical_keys)), "set_route_multi")

    def _set_routes(self, node_ids, keys, key_lens, lexical_keys, metadata) -> None:
        self._need_open()
        ids = np.ascontiguousarray(node_ids, dtype=np.uint64).reshape(-1)
        keys = np.ascontiguousarray(keys, dtype=np.float32).reshape(-1)
        lens = np.ascontiguousarray(key_lens, dtype=np.uint64).reshape(-1)
        lex = None
        if lexical_keys is not None:
            lex = (ctypes.c_char_p * ids.size)(*[_blob(x) for x in lexical_keys])
        meta = None
        if metadata is not None:
            flat = [str(v).encode("utf-8") if v else b"" for m in metadata for v in m]
            meta = (ctypes.c_char_p * (4 * ids.size))(*flat)
        self._check(self._lib.grm_hip_store_set_routes(
            self._h, ids.size, _ptr(ids), _ptr(keys), _ptr(lens),
            ctypes.cast(lex, ctypes.c_void_p) if lex is not None else None,
            ctypes.cast(meta, ctypes.c_void_p) if meta is not None else None), "set_routes")

    def set_route_metadata(self, node_id: int, kind="", scope="", durability="",
                           mutability="") -> None:
        """Non-empty values replace the entry's; a node without a route
        entry is left alone (cpp/grm_runtime.cpp:2922-2946)."""
        self._need_open()
        vals = [str(v).encode("utf-8") for v in (kind, scope, durability, mutability)]
        self._check(self._lib.grm_store_set_route_metadata(self._h, int(node_id), *vals),
                    "set_route_metadata")

    def clear_route(self, node_id: int) -> None:
        self._need_open()
        self._check(self._lib.grm_store_clear_route(self._h, int(node_id)), "clear_route")

    # --------------------------------------------------------------- route
    def _route_scored(self, q: np.ndarray, heads: int, tokens: int, lexical_keys, topk: int,
                      kinds, scopes, durabilities, mutabilities):
        self._need_open()
        k = int(topk)
        ids = np.empty(max(1, k), dtype=np.uint64)
        sc = np.empty(max(1, k), dtype=np.float32)
        count = ctypes.c_uint64(0)
        self._check(self._lib.grm_hip_store_route_scored(
            self._h, _ptr(q), heads, tokens, _blob(lexical_keys), _blob(kinds), _blob(scopes),
            _blob(durabilities), _blob(mutabilities), k, _ptr(ids), _ptr(sc), k,
            ctypes.byref(count)), "store route")
        n = int(count.value)
        return [int(x) for x in ids[:n]], [float(x) for x in sc[:n]]


class DeviceRouteStore(_Store):
    """MLA store route on the device.  Node ids are the store's.  ``route``
    / ``route_filtered`` return node ids like the reference ABI;
    ``route_scored`` also returns the route scores."""

    def __init__(self, dim: int, *, dtype: str = "f32", capacity: int = 1024):
        if dtype != "f32":
            raise ValueError("the store takes fp32 route keys")
        lib = _lib.load()
        h = ctypes.c_void_p()
        _lib.check(lib.grm_hip_store_create_mla(int(dim), max(64, int(capacity)),
                                                _lib.DTYPE_F32, ctypes.byref(h)),
                   "store create")
        super().__init__(h)
        self.dim = int(dim)

    def set_routes(self, node_ids, route_keys, lexical_keys=None, metadata=None) -> None:
        """Many new nodes at once.  lexical_keys[i] / metadata[i] (kind,
        scope, durability, mutability; empty values keep the defaults) may
        be omitted."""
        ids = np.ascontiguousarray(node_ids, dtype=np.uint64).reshape(-1)
        keys = np.ascontiguousarray(route_keys, dtype=np.float32).reshape(ids.size, -1)
        if keys.shape[1] != self.dim:
            raise ValueError("route keys do not match the store dim")
        self._set_routes(ids, keys, np.full(ids.size, self.dim, np.uint64), lexical_keys,
                         metadata)

    def route_scored(self, query, lexical_keys=(), topk: int = 3, *, kinds=(), scopes=(),
                     durabilities=(), mutabilities=()):
        """(node ids, route scores) of the store's route law, best first."""
        q = np.ascontiguousarray(query, dtype=np.float32).reshape(-1)
        if q.size != self.dim:
            raise ValueError("query dim does not match the store")
        return self._route_scored(q, 0, 0, lexical_keys, topk, kinds, scopes, durabilities,
                                  mutabilities)

    def route(self, query, lexical_keys=(), topk: int = 3) -> list[int]:
        """``grm_store_route``: node ids, best first."""
        self._need_open()
        q = np.ascontiguousarray(query, dtype=np.float32).reshape(-1)
        ids = np.empty(max(1, int(topk)), dtype=np.uint64)
        count = ctypes.c_uint64(0)
        self._check(self._lib.grm_store_route(self._h, _ptr(q), q.size, _blob(lexical_keys),
                                              int(topk), _ptr(ids), int(topk),
                                              ctypes.byref(count)), "grm_store_route")
        return [int(x) for x in ids[:count.value]]

    def route_filtered(self, query, lexical_keys=(), kinds=(), scopes=(), durabilities=(),
                       mutabilities=(), topk: int = 3) -> list[int]:
        """``grm_store_route_filtered``: node ids, best first."""
        self._need_open()
        q = np.ascontiguousarray(query, dtype=np.float32).reshape(-1)
        ids = np.empty(max(1, int(topk)), dtype=np.uint64)
        count = ctypes.c_uint64(0)
        self._check(self._lib.grm_store_route_filtered(
            self._h, _ptr(q), q.size, _blob(lexical_keys), _blob(kinds), _blob(scopes),
            _blob(durabilities), _blob(mutabilities), int(topk), _ptr(ids), int(topk),
            ctypes.byref(count)), "grm_store_route_filtered")
        return [int(x) for x in ids[:count.value]]


class DeviceGqaRouteStore(_Store):
    """GQA store route on the device (``grm_store_route_gqa``): route keys
    are [kv_heads][L][head_dim] fp32 blocks, queries [H][Qt][head_dim]."""

    def __init__(self, kv_heads: int, head_dim: int, *, capacity_nodes: int = 1024,
                 capacity_tokens: int = 1 << 16):
        lib = _lib.load()
        h = ctypes.c_void_p()
        _lib.check(lib.grm_hip_store_create_gqa(int(kv_heads), int(head_dim),
                                                int(capacity_nodes), int(capacity_tokens),
                                                ctypes.byref(h)), "store create")
        super().__init__(h)
        self.kv_heads = int(kv_heads)
        self.head_dim = int(head_dim)

    def set_routes(self, node_ids, blocks, lexical_keys=None, metadata=None) -> None:
        """Many new nodes at once: blocks[i] is node i's [kv][L_i][hd] key."""
        ids = np.ascontiguousarray(node_ids, dtype=np.uint64).reshape(-1)
        flat = [np.ascontiguousarray(b, dtype=np.float32).reshape(-1) for b in blocks]
        keys = np.concatenate(flat) if flat else np.zeros(0, np.float32)
        self._set_routes(ids, keys, [f.size for f in flat], lexical_keys, metadata)

    def route_scored(self, query, lexical_keys=(), topk: int = 3, *, kinds=(), scopes=(),
                     durabilities=(), mutabilities=()):
        """(node ids, route scores) of route_gqa_raw's law, best first:
        raw scores without lexical keys, normalised raw + bonus with them."""
        q = np.ascontiguousarray(query, dtype=np.float32)
        if q.ndim != 3 or q.shape[2] != self.head_dim:
            raise ValueError("query must be [H, Qt, head_dim]")
        return self._route_scored(q, q.shape[0], q.shape[1], lexical_keys, topk, kinds, scopes,
                                  durabilities, mutabilities)

    def route_gqa(self, query, lexical_keys=(), kinds=(), scopes=(), durabilities=(),
                  mutabilities=(), topk: int = 3) -> list[int]:
        """``grm_store_route_gqa``: node ids, best first."""
        self._need_open()
        q = np.ascontiguousarray(query, dtype=np.float32)
        if q.ndim != 3:
            raise ValueError("query must be [H, Qt, head_dim]")
        ids = np.empty(max(1, int(topk)), dtype=np.uint64)
        count = ctypes.c_uint64(0)
        self._check(self._lib.grm_store_route_gqa(
            self._h, _ptr(q), q.shape[0], q.shape[1], q.shape[2], _blob(lexical_keys),
            _blob(kinds), _blob(scopes), _blob(durabilities), _blob(mutabilities), int(topk),
            _ptr(ids), int(topk), ctypes.byref(count)), "grm_store_route_gqa")
        return [int(x) for x in ids[:count.value]]


__all__ = ["DeviceGqaRouteStore", "DeviceRouteStore", "filter_bits", "known_bit", "split_keys"]
