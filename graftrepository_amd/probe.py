"""One ctypes layer for both route dialects' reference sidecar entry points.

The reference binds each sidecar library through its own probe module
(scripts/grm_mla_cuda_probe.py:573-811, scripts/grm_gqa_cuda_probe.py:
632-911).  Callers see three objects there, and this module provides them
for either dialect from one table (:class:`Dialect`):

* a probe (``CudaProbe``): ``route_topk(bank, queries, *, warmup, topk)``
  one-shot, ``create_arena(bank)``, ``upload_queries(queries)``;
* an arena (``CudaDeviceArena``): ``route_topk(queries, *, warmup, topk)``,
  ``route_topk_device(device_queries, *, warmup, topk)``, ``close()``, the
  bank's sizes as attributes and ``setup_wall_ms``;
* a device query buffer (``CudaDeviceQueryPtr``): ``handle``, ``shape``,
  ``close()``.

Every route returns ``(row ids uint64 [Q, topk], device ms, wall ms)``:
device time from the ``warmup``-th query, wall time around the C call.
A nonzero return code raises ``RuntimeError`` naming the code; a query
whose last axis differs from the bank's, or topk above the node count,
raises ``ValueError``; a route on a closed arena raises ``RuntimeError``.
Inputs are taken as float32 C-contiguous copies when they are not already.
"""

from __future__ import annotations

import ctypes
import time
from dataclasses import dataclass
from typing import Callable

import numpy as np

from . import _lib


@dataclass(frozen=True)
class Dialect:
    """How one dialect's bank and queries map onto its C entry points.

    ``bank_axes`` names the bank array's axes (they become arena
    attributes); ``query_ndim`` is the query array's rank.  ``route_ints``
    gives the int arguments a route call takes between the query pointer
    and ``warmup``; ``oneshot_ints`` those the one-shot route takes between
    the query pointer and ``warmup``."""

    label: str
    symbol: str
    bank_axes: tuple[str, ...]
    query_ndim: int
    mismatch: str
    route_ints: Callable[[tuple, tuple], tuple]
    oneshot_ints: Callable[[tuple, tuple], tuple]

    def fn(self, lib, what: str):
        return getattr(lib, f"{self.symbol}_{what}")


# grm_mla_cuda_arena_route(arena, q, query_count, dim, warmup, topk, out, ms)
# grm_mla_cublas_route(rows, q, nodes, dim, query_count, warmup, topk, out, ms)
MLA = Dialect(
    label="MLA", symbol="grm_mla", bank_axes=("nodes", "dim"), query_ndim=2,
    mismatch="query dim does not match rows",
    route_ints=lambda bank, q: (q[0], bank[1]),
    oneshot_ints=lambda bank, q: (bank[0], bank[1], q[0]))

# grm_gqa_cuda_arena_route(arena, q, query_count, heads, tokens, warmup, ...)
# grm_gqa_cublas_route(keys, q, nodes, kv, key_tokens, query_count, heads,
#                      tokens, head_dim, warmup, ...)
GQA = Dialect(
    label="GQA", symbol="grm_gqa",
    bank_axes=("nodes", "kv_heads", "key_tokens", "head_dim"), query_ndim=4,
    mismatch="query head_dim does not match keys",
    route_ints=lambda bank, q: (q[0], q[1], q[2]),
    oneshot_ints=lambda bank, q: (bank[0], bank[1], bank[2], q[0], q[1], q[2], bank[3]))


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _checked_shape(d: Dialect, q_shape, bank_shape) -> tuple[int, ...]:
    q_shape = tuple(int(x) for x in q_shape)
    if len(q_shape) != d.query_ndim or q_shape[-1] != bank_shape[-1]:
        raise ValueError(d.mismatch)
    return q_shape


class _Call:
    """One C route call: output ids, the device-time cell, the wall clock."""

    def __init__(self, q_count: int, topk: int):
        self.ids = np.empty((q_count, topk), dtype=np.uint64)
        self.ms = ctypes.c_float(0.0)

    def run(self, fn, lead: tuple, ints: tuple, warmup: int, topk: int, what: str):
        t0 = time.perf_counter_ns()
        rc = fn(*lead, *ints, int(warmup), int(topk), self.ids.ctypes.data,
                ctypes.byref(self.ms))
        wall = (time.perf_counter_ns() - t0) / 1.0e6
        if rc != 0:
            raise RuntimeError(f"{what} failed with code {rc}")
        return self.ids, float(self.ms.value), wall


class DeviceQueryPtr:
    """Device query buffer from ``upload_queries``: ``handle`` (device
    address), ``shape``; freed by ``close()`` or collection."""

    def __init__(self, probe: "RouteProbe", handle: ctypes.c_void_p, *, shape):
        self.probe = probe
        self.handle = handle
        self.shape = tuple(int(x) for x in shape)

    def close(self) -> None:
        h, self.handle = getattr(self, "handle", None), ctypes.c_void_p()
        if h:
            self.probe.dialect.fn(self.probe.lib, "cuda_free_device_ptr")(h)

    __del__ = close


class ProbeArena:
    """A bank created on the device by ``RouteProbe.create_arena``."""

    def __init__(self, probe: "RouteProbe", handle: ctypes.c_void_p, *,
                 setup_wall_ms: float, **sizes):
        self.probe = probe
        self.handle = handle
        self.setup_wall_ms = setup_wall_ms
        self._shape = tuple(int(sizes[a]) for a in probe.dialect.bank_axes)
        for axis, n in zip(probe.dialect.bank_axes, self._shape):
            setattr(self, axis, n)

    def _destroy(self) -> int:
        h, self.handle = getattr(self, "handle", None), ctypes.c_void_p()
        return self.probe.dialect.fn(self.probe.lib, "cuda_arena_destroy")(h) if h else 0

    def close(self) -> None:
        rc = self._destroy()
        if rc != 0:
            raise RuntimeError(f"HIP {self.probe.dialect.label} arena destroy failed with code {rc}")

    def __del__(self) -> None:
        self._destroy()

    def _route(self, what: str, qptr, q_shape, warmup: int, topk: int):
        d = self.probe.dialect
        if not self.handle:
            raise RuntimeError(f"HIP {d.label} arena is closed")
        q_shape = _checked_shape(d, q_shape, self._shape)
        if topk > self._shape[0]:
            raise ValueError("topk cannot exceed node count")
        return _Call(q_shape[0], topk).run(
            d.fn(self.probe.lib, what), (self.handle, qptr), d.route_ints(self._shape, q_shape),
            warmup, topk, f"HIP {d.label} arena {what.replace('cuda_arena_', '')}")

    def route_topk(self, queries, *, warmup: int, topk: int):
        q = _f32(queries)
        return self._route("cuda_arena_route", q.ctypes.data, q.shape, warmup, topk)

    def route_topk_device(self, device_queries: DeviceQueryPtr, *, warmup: int, topk: int):
        return self._route("cuda_arena_route_device", device_queries.handle,
                           device_queries.shape, warmup, topk)


class RouteProbe:
    """The loaded route library seen through one dialect's sidecar entry
    points.  ``lib_path`` defaults to the in-tree library."""

    dialect: Dialect = MLA

    def __init__(self, lib_path=None, dialect: Dialect | None = None):
        if dialect is not None:
            self.dialect = dialect
        self.lib = _lib.load(lib_path)

    def upload_queries(self, queries) -> DeviceQueryPtr:
        q = _f32(queries)
        handle = ctypes.c_void_p()
        rc = self.dialect.fn(self.lib, "cuda_upload_queries")(
            q.ctypes.data, ctypes.c_size_t(q.size), ctypes.byref(handle))
        if rc != 0:
            raise RuntimeError(f"HIP query upload failed with code {rc}")
        return DeviceQueryPtr(self, handle, shape=q.shape)

    def route_topk(self, bank, queries, *, warmup: int, topk: int):
        d = self.dialect
        b, q = _f32(bank), _f32(queries)
        q_shape = _checked_shape(d, q.shape, b.shape)
        return _Call(q_shape[0], topk).run(
            d.fn(self.lib, "cublas_route"), (b.ctypes.data, q.ctypes.data),
            d.oneshot_ints(b.shape, q_shape), warmup, topk, f"HIP {d.label} probe")

    def create_arena(self, bank) -> ProbeArena:
        d = self.dialect
        b = _f32(bank)
        if b.ndim != len(d.bank_axes):
            raise ValueError(f"{d.label} bank must have axes {d.bank_axes}")
        handle = ctypes.c_void_p()
        t0 = time.perf_counter_ns()
        rc = d.fn(self.lib, "cuda_arena_create")(b.ctypes.data, *b.shape, ctypes.byref(handle))
        setup = (time.perf_counter_ns() - t0) / 1.0e6
        if rc != 0:
            raise RuntimeError(f"HIP {d.label} arena create failed with code {rc}")
        return ProbeArena(self, handle, setup_wall_ms=setup, **dict(zip(d.bank_axes, b.shape)))
