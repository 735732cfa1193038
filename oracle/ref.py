"""ctypes binding of the reference's CPU router built into ``oracle/_ref``.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  The library is the
reference's ``cpp/grm_runtime.cpp`` compiled from its sources by
``oracle/Makefile`` (target ``ref``); this module drives its store C ABI
(``cpp/grm_runtime_c.h:70-499``) to produce route orders for golden fixtures
and for pinning the oracle restatement.

Route entry points used:
  grm_store_route      cpp/grm_runtime.cpp:6767-6825 -> route_mla_arena (fp64)
  grm_store_route_filtered  cpp/grm_runtime.cpp:6840-6897 -> route_mla_arena
                       with lexical bonus and route filters
  grm_store_route_gqa  cpp/grm_runtime.cpp:6898-6961 -> route_gqa_raw
``route_gqa_raw`` takes its fp32 arena path when every route key's length is
a multiple of kv_heads*head_dim, and the fp64 ``gqa_raw_score`` path
otherwise (cpp/grm_runtime.cpp:3321-3327, 4775-4800).  ``fp64_gqa=True``
adds one extra node whose single-value key makes the arena invalid, forcing
the fp64 law; that node scores 0.0 (cpp/grm_runtime.cpp:2998-3001) and is
dropped from the returned order.
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import REF_LIB_PATH, build_ref

_ref = None


def available() -> bool:
    return REF_LIB_PATH.exists() or build_ref() is not None


def lib() -> ctypes.CDLL:
    global _ref
    if _ref is None:
        path = REF_LIB_PATH if REF_LIB_PATH.exists() else build_ref()
        if path is None or not path.exists():
            raise FileNotFoundError("reference CPU router not built")
        L = ctypes.CDLL(str(path))
        vp, u64, i32, cp = (ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int,
                            ctypes.c_char_p)
        L.grm_store_create_mla.argtypes = [cp, i32, i32, i32, i32, i32, i32]
        L.grm_store_create_mla.restype = vp
        L.grm_store_create_gqa.argtypes = [cp, i32, i32, i32, i32, i32, i32]
        L.grm_store_create_gqa.restype = vp
        L.grm_store_destroy.argtypes = [vp]
        L.grm_store_destroy.restype = None
        L.grm_store_add_node.argtypes = [vp, cp, u64, vp, u64,
                                         ctypes.POINTER(u64)]
        L.grm_store_add_node.restype = i32
        L.grm_store_set_route.argtypes = [vp, u64, vp, u64, cp]
        L.grm_store_set_route.restype = i32
        L.grm_store_set_route_list.argtypes = [vp, u64, vp, u64, vp, u64, cp]
        L.grm_store_set_route_list.restype = i32
        L.grm_store_route.argtypes = [vp, vp, u64, cp, u64, vp, u64,
                                      ctypes.POINTER(u64)]
        L.grm_store_route.restype = i32
        L.grm_store_route_gqa.argtypes = [vp, vp, u64, u64, u64, cp, cp, cp,
                                          cp, cp, u64, vp, u64,
                                          ctypes.POINTER(u64)]
        L.grm_store_route_gqa.restype = i32
        L.grm_store_last_error.argtypes = [vp]
        L.grm_store_last_error.restype = cp
        L.grm_store_set_route_metadata.argtypes = [vp, u64, cp, cp, cp, cp]
        L.grm_store_set_route_metadata.restype = i32
        L.grm_store_route_filtered.argtypes = [vp, vp, u64, cp, cp, cp, cp, cp, u64, vp, u64,
                                               ctypes.POINTER(u64)]
        L.grm_store_route_filtered.restype = i32
        _ref = L
    return _ref


class _Store:
    def __init__(self, handle):
        if not handle:
            raise RuntimeError("reference store create failed")
        self.h = handle

    def close(self):
        if self.h:
            lib().grm_store_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def _check(self, rc):
        if rc != 0:
            err = lib().grm_store_last_error(self.h)
            raise RuntimeError(f"reference store error {rc}: {err!r}")

    def add_node(self) -> int:
        out = ctypes.c_uint64()
        self._check(lib().grm_store_add_node(self.h, b"n", 1, None, 0,
                                             ctypes.byref(out)))
        return int(out.value)

    def set_route(self, node_id: int, key: np.ndarray):
        k = np.ascontiguousarray(key, dtype=np.float32).reshape(-1)
        self._check(lib().grm_store_set_route(self.h, node_id, k.ctypes.data,
                                              k.size, b""))

    def set_route_list(self, node_id: int, keys: list[np.ndarray], lexical: bytes = b""):
        flat = [np.ascontiguousarray(k, dtype=np.float32).reshape(-1)
                for k in keys]
        values = (np.concatenate(flat) if flat
                  else np.zeros(0, dtype=np.float32))
        offs = np.zeros(len(flat) + 1, dtype=np.uint64)
        offs[1:] = np.cumsum([f.size for f in flat])
        self._check(lib().grm_store_set_route_list(
            self.h, node_id, values.ctypes.data, values.size,
            offs.ctypes.data, len(flat), lexical))


def _keys_of(entry, row_len: int | None = None) -> list:
    """An entry's route keys: one array, or a list / 2-D stack of them."""
    if isinstance(entry, (list, tuple)):
        return [np.asarray(k, dtype=np.float32) for k in entry]
    a = np.asarray(entry, dtype=np.float32)
    if row_len is not None and a.ndim == 2:
        return [a[i] for i in range(a.shape[0])]
    return [a]


def _blob(items) -> bytes:
    return "\n".join(items).encode("utf-8")


def store_route(rows, lexical: list, meta: list, query: np.ndarray,
                query_lexical=(), filters=((), (), (), ()), topk: int = 3) -> list[int]:
    """Route order from the reference ``grm_store_route_filtered``
    (cpp/grm_runtime.cpp:6840-6897 -> route_mla_arena): node i has route
    key rows[i] (one row; a 2-D stack or a list of rows makes a multi-row
    entry, set through grm_store_set_route_list), lexical keys lexical[i]
    and route metadata meta[i] = (kind, scope, durability, mutability).
    filters = (kinds, scopes, durabilities, mutabilities), each a list of
    values."""
    q = np.ascontiguousarray(query, dtype=np.float32).reshape(-1)
    d = q.size
    h = lib().grm_store_create_mla(b"MiniCPM3_TC", 62, 2560, d, 0, d, 0)
    with _Store(h) as st:
        for i in range(len(rows)):
            nid = st.add_node()
            assert nid == i
            keys = _keys_of(rows[i], d)
            if len(keys) == 1:
                k = np.ascontiguousarray(keys[0]).reshape(-1)
                st._check(lib().grm_store_set_route(st.h, nid, k.ctypes.data, k.size,
                                                    _blob(lexical[i])))
            else:
                st.set_route_list(nid, keys, _blob(lexical[i]))
            st._check(lib().grm_store_set_route_metadata(
                st.h, nid, *[str(v).encode("utf-8") for v in meta[i]]))
        out = np.empty(max(1, topk), dtype=np.uint64)
        count = ctypes.c_uint64()
        st._check(lib().grm_store_route_filtered(
            st.h, q.ctypes.data, q.size, _blob(query_lexical), *[_blob(f) for f in filters],
            topk, out.ctypes.data, topk, ctypes.byref(count)))
        return [int(x) for x in out[:count.value]]


def mla_route(rows: np.ndarray, query: np.ndarray, topk: int) -> list[int]:
    """Route order from the reference ``grm_store_route`` (node id = row)."""
    r = np.ascontiguousarray(rows, dtype=np.float32)
    q = np.ascontiguousarray(query, dtype=np.float32).reshape(-1)
    d = r.shape[1]
    h = lib().grm_store_create_mla(b"MiniCPM3_TC", 62, 2560, d, 0, d, 0)
    with _Store(h) as st:
        for i in range(r.shape[0]):
            nid = st.add_node()
            assert nid == i
            st.set_route(nid, r[i])
        out = np.empty(max(1, topk), dtype=np.uint64)
        count = ctypes.c_uint64()
        st._check(lib().grm_store_route(st.h, q.ctypes.data, q.size, b"",
                                        topk, out.ctypes.data, topk,
                                        ctypes.byref(count)))
        return [int(x) for x in out[:count.value]]


def gqa_route(node_keys: list, query: np.ndarray, kv_heads: int, topk: int,
              *, fp64_gqa: bool = True) -> list[int]:
    """Route order from the reference ``grm_store_route_gqa``.

    ``node_keys[i]`` is either one array [KV, L, hd] or a list of such arrays
    (a multi-key node).  Node id = list index.
    """
    q = np.ascontiguousarray(query, dtype=np.float32)
    H, Qt, hd = q.shape
    h = lib().grm_store_create_gqa(b"Qwen3_TC", 36, 2560, 2 * kv_heads * hd, 0,
                                   kv_heads, hd)
    with _Store(h) as st:
        for i, key in enumerate(node_keys):
            nid = st.add_node()
            assert nid == i
            keys = key if isinstance(key, (list, tuple)) else [key]
            st.set_route_list(nid, list(keys))
        sentinel = None
        if fp64_gqa:
            sentinel = st.add_node()
            st.set_route(sentinel, np.zeros(1, dtype=np.float32))
        want = topk + (1 if fp64_gqa else 0)
        out = np.empty(max(1, want), dtype=np.uint64)
        count = ctypes.c_uint64()
        st._check(lib().grm_store_route_gqa(
            st.h, q.ctypes.data, H, Qt, hd, b"", b"", b"", b"", b"", want,
            out.ctypes.data, want, ctypes.byref(count)))
        order = [int(x) for x in out[:count.value]]
        if sentinel is not None:
            order = [x for x in order if x != sentinel]
        return order[:topk]


def store_route_gqa(blocks: list, lexical: list, meta: list, query: np.ndarray, kv_heads: int,
                    query_lexical=(), filters=((), (), (), ()), topk: int = 3) -> list[int]:
    """Route order from the reference ``grm_store_route_gqa`` with lexical
    keys and route filters: node i (id i) has key blocks[i] [kv, L, hd] (a
    list of such blocks makes a multi-key entry), lexical keys lexical[i]
    and metadata meta[i].  A sentinel node with a one-value key keeps the
    store on its fp64 law path (see gqa_route) and is dropped from the
    order."""
    q = np.ascontiguousarray(query, dtype=np.float32)
    H, Qt, hd = q.shape
    h = lib().grm_store_create_gqa(b"Qwen3_TC", 36, 2560, 2 * kv_heads * hd, 0, kv_heads, hd)
    with _Store(h) as st:
        for i, key in enumerate(blocks):
            nid = st.add_node()
            assert nid == i
            st.set_route_list(nid, _keys_of(key), _blob(lexical[i]))
            st._check(lib().grm_store_set_route_metadata(
                st.h, nid, *[str(v).encode("utf-8") for v in meta[i]]))
        sentinel = st.add_node()
        st.set_route(sentinel, np.zeros(1, dtype=np.float32))
        want = topk + 1
        out = np.empty(want, dtype=np.uint64)
        count = ctypes.c_uint64()
        st._check(lib().grm_store_route_gqa(
            st.h, q.ctypes.data, H, Qt, hd, _blob(query_lexical), *[_blob(f) for f in filters],
            want, out.ctypes.data, want, ctypes.byref(count)))
        order = [int(x) for x in out[:count.value] if int(x) != sentinel]
        return order[:topk]
