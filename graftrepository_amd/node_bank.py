"""Device-resident node banks: the library's extended route API.

``MlaNodeBank`` and ``GqaNodeBank`` own a bank on the current HIP device and
return node ids *and* scores (the reference sidecar returns row ids only,
core/grm_cuda_router.py:183-231).  Both support append and evict through the
bank's side stream, replacing the reference's full rebuild and re-upload on
every arena mutation (core/graft_arena.py:1164-1198, 2979-3042).

Inputs are numpy arrays.  bf16 data is passed as uint16 bit patterns (see
``as_bf16_bits``); int8 GQA banks take codes plus per-(token, group) scales.
Device-resident queries can be passed as any object with a ``data_ptr()``
method (e.g. a torch tensor) or an integer device address.
"""

from __future__ import annotations

import ctypes
import time
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import DTYPE_BF16, DTYPE_CODES, DTYPE_F16, DTYPE_F32, DTYPE_I8


def as_bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns (uint16), round to nearest even."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = np.isnan(np.ascontiguousarray(x, dtype=np.float32))
    r = ((u + (np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))))
         >> np.uint32(16)).astype(np.uint16)
    if np.any(nan):
        r[nan] = ((u[nan] >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16)
    return r.reshape(np.shape(x))


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32)
            << np.uint32(16)).view(np.float32)


def _dtype_code(dtype) -> int:
    if isinstance(dtype, int):
        return dtype
    return DTYPE_CODES[str(dtype)]


def _ptr(a) -> int | None:
    if a is None:
        return None
    return a.ctypes.data


def _device_ptr(obj) -> int:
    if isinstance(obj, int):
        return obj
    if hasattr(obj, "data_ptr"):
        return int(obj.data_ptr())
    if hasattr(obj, "handle"):
        h = obj.handle
        return int(h.value if isinstance(h, ctypes.c_void_p) else h)
    raise TypeError("device queries need data_ptr(), .handle or an address")


def _device_nbytes(obj) -> int | None:
    """Bytes a device query object holds, when it says (``nbytes``, or a
    torch tensor's element count and size); None for a bare address."""
    if isinstance(obj, int):
        return None
    nb = getattr(obj, "nbytes", None)
    if isinstance(nb, int):
        return nb
    numel, esz = getattr(obj, "numel", None), getattr(obj, "element_size", None)
    if callable(numel) and callable(esz):
        return int(numel()) * int(esz())
    return None


@dataclass(frozen=True)
class RouteResult:
    """Top-k per query: node ids (UINT64_MAX = unfilled), scores (NaN =
    unfilled), device milliseconds from the warmup-th query, wall ms."""
    ids: np.ndarray
    scores: np.ndarray
    device_ms: float
    wall_ms: float


class _Bank:
    _destroy_name = ""

    def __init__(self):
        self._lib = _lib.load()
        self._h = ctypes.c_void_p()

    def close(self) -> None:
        if self._h:
            getattr(self._lib, self._destroy_name)(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def _need_open(self):
        if not self._h:
            raise RuntimeError("bank is closed")


class MlaNodeBank(_Bank):
    """MLA latent-centroid bank: one row of ``dim`` values per node."""

    _destroy_name = "grm_mla_cuda_arena_destroy"

    def __init__(self, rows: np.ndarray | None, node_ids=None, *,
                 dtype: str = "f32", dim: int | None = None,
                 capacity: int = 0):
        super().__init__()
        self.dtype = _dtype_code(dtype)
        if self.dtype not in (DTYPE_F32, DTYPE_BF16):
            raise ValueError("MLA banks store f32 or bf16")
        rows_np = self._rows(rows, dim)
        n, d = rows_np.shape
        ids = None
        if node_ids is not None:
            ids = np.ascontiguousarray(node_ids, dtype=np.uint64).reshape(-1)
            if ids.size != n:
                raise ValueError("node_ids length must match rows")
        self.dim = int(d)
        rc = self._lib.grm_mla_hip_bank_create(
            _ptr(rows_np) if n else None, self.dtype, n, self.dim, _ptr(ids),
            int(capacity), ctypes.byref(self._h))
        _lib.check(rc, "MLA bank create")

    def _rows(self, rows, dim) -> np.ndarray:
        want = np.float32 if self.dtype == DTYPE_F32 else np.uint16
        if rows is None:
            if dim is None:
                raise ValueError("dim is required for an empty bank")
            return np.zeros((0, int(dim)), dtype=want)
        r = np.asarray(rows)
        if self.dtype == DTYPE_BF16 and r.dtype != np.uint16:
            r = as_bf16_bits(r)
        r = np.ascontiguousarray(r, dtype=want)
        if r.ndim != 2:
            raise ValueError("rows must have shape (nodes, dim)")
        return r

    def route(self, queries, topk: int, *, warmup: int = 0,
              on_device: bool = False, query_dtype: str | None = None,
              query_count: int | None = None, timed: bool = True) -> RouteResult:
        """Route queries [Q, dim] (or [dim]); returns ids/scores [Q, topk].
        With ``timed=False`` no device time is taken (``device_ms`` is NaN)
        and the library may report completion without a stream event."""
        self._need_open()
        qd = self.dtype if query_dtype is None else _dtype_code(query_dtype)
        if on_device:
            qptr = _device_ptr(queries)
            if query_count is None:
                shape = getattr(queries, "shape", None)
                query_count = int(shape[0]) if shape is not None and len(shape) == 2 else 1
            q_count = int(query_count)
            need = q_count * self.dim * (4 if qd == DTYPE_F32 else 2)
            have = _device_nbytes(queries)
            if have is not None and have < need:
                raise ValueError(f"device queries hold {have} bytes, {q_count} queries need {need}")
            keep = None
        else:
            q = np.asarray(queries)
            if qd == DTYPE_BF16 and q.dtype != np.uint16:
                q = as_bf16_bits(q)
            q = np.ascontiguousarray(q, dtype=np.float32 if qd == DTYPE_F32 else np.uint16)
            if q.ndim == 1:
                q = q[None]
            if q.ndim != 2 or q.shape[1] != self.dim:
                raise ValueError("queries must have shape (Q, dim)")
            q_count = q.shape[0]
            qptr = _ptr(q)
            keep = q
        ids = np.empty((q_count, topk), dtype=np.uint64)
        scores = np.empty((q_count, topk), dtype=np.float32)
        ms = ctypes.c_float(0.0)
        t0 = time.perf_counter_ns()
        rc = self._lib.grm_mla_hip_route(
            self._h, qptr, qd, 1 if on_device else 0, q_count, self.dim,
            int(warmup), int(topk), _ptr(ids), _ptr(scores),
            ctypes.byref(ms) if timed else None)
        wall = (time.perf_counter_ns() - t0) / 1e6
        del keep
        _lib.check(rc, "MLA route")
        return RouteResult(ids, scores, float(ms.value) if timed else float("nan"), wall)

    def probe_screen(self, queries, *, query_dtype: str = "bf16"):
        """Test entry: the batched route's screened score of every (query,
        slot) pair of a small bf16 bank and each query's screen bound B.
        Returns (values [Q, slots] f32, bounds [Q] f64, slot node ids)."""
        self._need_open()
        qd = _dtype_code(query_dtype)
        q = np.asarray(queries)
        if qd == DTYPE_BF16 and q.dtype != np.uint16:
            q = as_bf16_bits(q)
        q = np.ascontiguousarray(q, dtype=np.float32 if qd == DTYPE_F32 else np.uint16)
        if q.ndim != 2 or q.shape[1] != self.dim:
            raise ValueError("queries must have shape (Q, dim)")
        n = int(self.info()["slots_in_use"])
        vals = np.empty((q.shape[0], n), dtype=np.float32)
        bounds = np.empty(q.shape[0], dtype=np.float64)
        ids = np.empty(n, dtype=np.uint64)
        _lib.check(self._lib.grm_mla_hip_probe_screen(self._h, _ptr(q), qd, q.shape[0], _ptr(vals),
                                                      _ptr(bounds), _ptr(ids)), "MLA probe screen")
        return vals, bounds, ids

    def latent_query(self, latent, tokens: int, *, dtype: str = "f16",
                     row_stride: int = 0, normalize: bool = True, out=None) -> int:
        """Write the route key of a device latent block [tokens][dim]
        (core/kv_graft.py:131-142) to device memory ``out`` (a device
        address or an object with ``data_ptr()``; dim floats)."""
        self._need_open()
        _lib.check(self._lib.grm_mla_hip_latent_query(
            self._h, _device_ptr(latent), _dtype_code(dtype), int(tokens), int(row_stride),
            1 if normalize else 0, _device_ptr(out)), "MLA latent query")
        return _device_ptr(out)

    def route_latent(self, latent, tokens: int, topk: int, *, dtype: str = "f16",
                     row_stride: int = 0, timed: bool = True) -> RouteResult:
        """Route the key of a device latent block without a host round
        trip: the key is formed on the route stream and routed there.
        ``timed=False`` as in ``route``."""
        self._need_open()
        ids = np.empty((1, topk), dtype=np.uint64)
        scores = np.empty((1, topk), dtype=np.float32)
        ms = ctypes.c_float(0.0)
        t0 = time.perf_counter_ns()
        rc = self._lib.grm_mla_hip_route_latent(
            self._h, _device_ptr(latent), _dtype_code(dtype), int(tokens), int(row_stride),
            int(topk), _ptr(ids), _ptr(scores), ctypes.byref(ms) if timed else None)
        wall = (time.perf_counter_ns() - t0) / 1e6
        _lib.check(rc, "MLA latent route")
        return RouteResult(ids, scores, float(ms.value) if timed else float("nan"), wall)

    def score_nodes(self, query, node_ids, *, query_dtype: str = "f32") -> np.ndarray:
        """Exact law scores (float32, NaN where not finite) of the listed
        live node ids for one host query [dim]."""
        self._need_open()
        qd = _dtype_code(query_dtype)
        q = np.asarray(query)
        if qd == DTYPE_BF16 and q.dtype != np.uint16:
            q = as_bf16_bits(q)
        q = np.ascontiguousarray(q, dtype=np.float32 if qd == DTYPE_F32 else np.uint16).reshape(-1)
        if q.size != self.dim:
            raise ValueError("query must have dim values")
        ids = np.ascontiguousarray(node_ids, dtype=np.uint64).reshape(-1)
        out = np.empty(ids.size, dtype=np.float32)
        _lib.check(self._lib.grm_mla_hip_score_nodes(self._h, _ptr(q), qd, _ptr(ids), ids.size,
                                                     _ptr(out)), "MLA score nodes")
        return out

    def append(self, rows, node_ids) -> int:
        self._need_open()
        r = self._rows(rows, self.dim)
        ids = np.ascontiguousarray(node_ids, dtype=np.uint64).reshape(-1)
        if ids.size != r.shape[0] or r.shape[1] != self.dim:
            raise ValueError("rows/node_ids shape mismatch")
        epoch = ctypes.c_uint64()
        rc = self._lib.grm_mla_hip_append(self._h, _ptr(r), self.dtype,
                                          r.shape[0], _ptr(ids),
                                          ctypes.byref(epoch))
        _lib.check(rc, "MLA append")
        return int(epoch.value)

    def evict(self, node_ids) -> int:
        self._need_open()
        ids = np.ascontiguousarray(node_ids, dtype=np.uint64).reshape(-1)
        epoch = ctypes.c_uint64()
        rc = self._lib.grm_mla_hip_evict(self._h, _ptr(ids), ids.size,
                                         ctypes.byref(epoch))
        _lib.check(rc, "MLA evict")
        return int(epoch.value)

    def sync(self) -> None:
        self._need_open()
        _lib.check(self._lib.grm_mla_hip_sync(self._h), "MLA sync")

    def info(self) -> dict:
        self._need_open()
        out = np.zeros(6, dtype=np.uint64)
        _lib.check(self._lib.grm_mla_hip_bank_info(self._h, _ptr(out)),
                   "MLA info")
        keys = ("live", "capacity", "slots_in_use", "epoch", "dim", "dtype")
        return {k: int(v) for k, v in zip(keys, out)}

    def route_stats(self) -> dict:
        """Counters since create: batched (matrix-core) queries, their
        fallbacks to the single-query kernel, single-kernel queries, passes."""
        self._need_open()
        out = np.zeros(4, dtype=np.uint64)
        _lib.check(self._lib.grm_mla_hip_route_stats(self._h, _ptr(out)),
                   "MLA route stats")
        keys = ("batched", "fallbacks", "single", "passes")
        return {k: int(v) for k, v in zip(keys, out)}

    def screen_ms(self) -> float:
        """Device time of the matrix-core screen kernels in the timed part
        of the last route (0.0 when it did not take the batched path)."""
        self._need_open()
        out = np.zeros(1, dtype=np.float32)
        _lib.check(self._lib.grm_mla_hip_screen_ms(self._h, _ptr(out)),
                   "MLA screen time")
        return float(out[0])


class GqaNodeBank(_Bank):
    """Ragged GQA bank: node i has a key block [kv_heads, L_i, head_dim]."""

    _destroy_name = "grm_gqa_cuda_arena_destroy"

    def __init__(self, keys, tok_offsets, *, kv_heads: int, head_dim: int,
                 node_ids=None, dtype: str = "f32", scales=None,
                 scale_dtype: str = "f32", group_size: int = 0,
                 capacity_nodes: int = 0, capacity_tokens: int = 0):
        super().__init__()
        self.dtype = _dtype_code(dtype)
        self.scale_dtype = _dtype_code(scale_dtype)
        self.kv_heads = int(kv_heads)
        self.head_dim = int(head_dim)
        self.group_size = int(group_size)
        offs = np.ascontiguousarray(tok_offsets, dtype=np.uint64).reshape(-1)
        n = offs.size - 1
        k = self._keys(keys)
        s = self._scales(scales)
        ids = None
        if node_ids is not None:
            ids = np.ascontiguousarray(node_ids, dtype=np.uint64).reshape(-1)
            if ids.size != n:
                raise ValueError("node_ids length must match nodes")
        rc = self._lib.grm_gqa_hip_bank_create(
            _ptr(k), self.dtype, _ptr(s), self.scale_dtype, self.group_size,
            _ptr(offs), n, self.kv_heads, self.head_dim, _ptr(ids),
            int(capacity_nodes), int(capacity_tokens), ctypes.byref(self._h))
        _lib.check(rc, "GQA bank create")

    def _keys(self, keys):
        if keys is None:
            return None
        k = np.asarray(keys)
        if self.dtype == DTYPE_F32:
            return np.ascontiguousarray(k, dtype=np.float32).reshape(-1)
        if self.dtype == DTYPE_BF16:
            if k.dtype != np.uint16:
                k = as_bf16_bits(k)
            return np.ascontiguousarray(k, dtype=np.uint16).reshape(-1)
        if self.dtype == DTYPE_F16:
            if k.dtype != np.uint16:
                k = np.ascontiguousarray(k, dtype=np.float16).view(np.uint16)
            return np.ascontiguousarray(k, dtype=np.uint16).reshape(-1)
        return np.ascontiguousarray(k, dtype=np.int8).reshape(-1)

    def _scales(self, scales):
        if self.dtype != DTYPE_I8:
            return None
        if scales is None:
            raise ValueError("int8 banks need scales")
        s = np.asarray(scales)
        if self.scale_dtype == DTYPE_F16:
            if s.dtype != np.uint16:
                s = np.ascontiguousarray(s, dtype=np.float16).view(np.uint16)
            return np.ascontiguousarray(s, dtype=np.uint16).reshape(-1)
        return np.ascontiguousarray(s, dtype=np.float32).reshape(-1)

    def route(self, queries, topk: int, *, warmup: int = 0,
              on_device: bool = False, query_dtype: str = "f32",
              query_shape: tuple[int, int, int, int] | None = None,
              timed: bool = True) -> RouteResult:
        """Route queries [Q, H, Qt, hd] (or [H, Qt, hd]).  With
        ``timed=False`` no device time is taken (``device_ms`` is NaN) and
        the library may report completion without a stream event."""
        self._need_open()
        qd = _dtype_code(query_dtype)
        if on_device:
            if query_shape is None:
                query_shape = tuple(int(x) for x in queries.shape)
            if len(query_shape) == 3:
                query_shape = (1, *query_shape)
            if len(query_shape) != 4 or query_shape[3] != self.head_dim:
                raise ValueError("query_shape must be (Q, H, Qt, head_dim)")
            need = int(np.prod(query_shape, dtype=np.int64)) * (4 if qd == DTYPE_F32 else 2)
            have = _device_nbytes(queries)
            if have is not None and have < need:
                raise ValueError(f"device queries hold {have} bytes, the shape needs {need}")
            qptr = _device_ptr(queries)
            keep = None
        else:
            q = np.asarray(queries)
            if qd == DTYPE_BF16 and q.dtype != np.uint16:
                q = as_bf16_bits(q)
            q = np.ascontiguousarray(q, dtype=np.float32 if qd == DTYPE_F32 else np.uint16)
            if q.ndim == 3:
                q = q[None]
            if q.ndim != 4 or q.shape[3] != self.head_dim:
                raise ValueError("queries must have shape (Q, H, Qt, head_dim)")
            query_shape = q.shape
            qptr = _ptr(q)
            keep = q
        qc, H, Qt, _ = query_shape
        ids = np.empty((qc, topk), dtype=np.uint64)
        scores = np.empty((qc, topk), dtype=np.float32)
        ms = ctypes.c_float(0.0)
        t0 = time.perf_counter_ns()
        rc = self._lib.grm_gqa_hip_route(
            self._h, qptr, qd, 1 if on_device else 0, qc, H, Qt, int(warmup),
            int(topk), _ptr(ids), _ptr(scores), ctypes.byref(ms) if timed else None)
        wall = (time.perf_counter_ns() - t0) / 1e6
        del keep
        _lib.check(rc, "GQA route")
        return RouteResult(ids, scores, float(ms.value) if timed else float("nan"), wall)

    def probe_screen(self, query, *, query_dtype: str = "bf16"):
        """Test entry: the bound-and-verify screen of one query [H, Qt, hd].
        Returns (maxima [slots, kv, R*Qt] f32 in the screen's scaled units,
        colinfo [kv, R*Qt, 4] = (coef, eabs, scale, kcap), K [slots] f64,
        slot node ids)."""
        self._need_open()
        qd = _dtype_code(query_dtype)
        q = np.asarray(query)
        if qd == DTYPE_BF16 and q.dtype != np.uint16:
            q = as_bf16_bits(q)
        q = np.ascontiguousarray(q, dtype=np.float32 if qd == DTYPE_F32 else np.uint16)
        if q.ndim != 3 or q.shape[2] != self.head_dim:
            raise ValueError("query must have shape (H, Qt, head_dim)")
        H, Qt, _ = q.shape
        cols = H // self.kv_heads * Qt
        n = int(self.info()["capacity_nodes"])
        maxima = np.empty((n, self.kv_heads, cols), dtype=np.float32)
        colinfo = np.empty((self.kv_heads, cols, 4), dtype=np.float32)
        knorm = np.empty(n, dtype=np.float64)
        ids = np.empty(n, dtype=np.uint64)
        _lib.check(self._lib.grm_gqa_hip_probe_screen(self._h, _ptr(q), qd, H, Qt, _ptr(maxima),
                                                      _ptr(colinfo), _ptr(knorm), _ptr(ids)),
                   "GQA probe screen")
        return maxima, colinfo, knorm, ids

    def score_nodes(self, query, node_ids, *, query_dtype: str = "f32") -> np.ndarray:
        """Exact raw law scores (float32, NaN where not finite) of the
        listed live node ids for one host query [H, Qt, hd]."""
        self._need_open()
        qd = _dtype_code(query_dtype)
        q = np.asarray(query)
        if qd == DTYPE_BF16 and q.dtype != np.uint16:
            q = as_bf16_bits(q)
        q = np.ascontiguousarray(q, dtype=np.float32 if qd == DTYPE_F32 else np.uint16)
        if q.ndim != 3 or q.shape[2] != self.head_dim:
            raise ValueError("query must have shape (H, Qt, head_dim)")
        ids = np.ascontiguousarray(node_ids, dtype=np.uint64).reshape(-1)
        out = np.empty(ids.size, dtype=np.float32)
        _lib.check(self._lib.grm_gqa_hip_score_nodes(self._h, _ptr(q), qd, q.shape[0], q.shape[1],
                                                     _ptr(ids), ids.size, _ptr(out)),
                   "GQA score nodes")
        return out

    def append(self, keys, tok_counts, node_ids, scales=None) -> int:
        self._need_open()
        k = self._keys(keys)
        s = self._scales(scales) if self.dtype == DTYPE_I8 else None
        counts = np.ascontiguousarray(tok_counts, dtype=np.uint64).reshape(-1)
        ids = np.ascontiguousarray(node_ids, dtype=np.uint64).reshape(-1)
        if ids.size != counts.size:
            raise ValueError("tok_counts and node_ids differ in length")
        epoch = ctypes.c_uint64()
        rc = self._lib.grm_gqa_hip_append(self._h, _ptr(k), _ptr(s),
                                          _ptr(counts), counts.size, _ptr(ids),
                                          ctypes.byref(epoch))
        _lib.check(rc, "GQA append")
        return int(epoch.value)

    def evict(self, node_ids) -> int:
        self._need_open()
        ids = np.ascontiguousarray(node_ids, dtype=np.uint64).reshape(-1)
        epoch = ctypes.c_uint64()
        rc = self._lib.grm_gqa_hip_evict(self._h, _ptr(ids), ids.size,
                                         ctypes.byref(epoch))
        _lib.check(rc, "GQA evict")
        return int(epoch.value)

    def compact(self) -> None:
        self._need_open()
        _lib.check(self._lib.grm_gqa_hip_compact(self._h), "GQA compact")

    def sync(self) -> None:
        self._need_open()
        _lib.check(self._lib.grm_gqa_hip_sync(self._h), "GQA sync")

    def info(self) -> dict:
        self._need_open()
        out = np.zeros(8, dtype=np.uint64)
        _lib.check(self._lib.grm_gqa_hip_bank_info(self._h, _ptr(out)),
                   "GQA info")
        keys = ("live", "capacity_nodes", "tokens_in_use", "capacity_tokens",
                "epoch", "kv_heads", "head_dim", "dtype")
        return {k: int(v) for k, v in zip(keys, out)}

    def route_stats(self) -> dict:
        """Counters since create: route calls, query passes screened and
        refined, passes bound and verified, queries routed exactly."""
        self._need_open()
        out = np.zeros(4, dtype=np.uint64)
        _lib.check(self._lib.grm_gqa_hip_route_stats(self._h, _ptr(out)), "GQA route stats")
        keys = ("routes", "screen_refine", "bound_verify", "exact")
        return {k: int(v) for k, v in zip(keys, out)}


__all__ = ["MlaNodeBank", "GqaNodeBank", "RouteResult", "as_bf16_bits",
           "bf16_bits_to_f32", "DTYPE_F32", "DTYPE_BF16", "DTYPE_F16",
           "DTYPE_I8"]
