"""Host binding of the MLA route library, mirroring the reference probe's
ctypes layer (scripts/grm_mla_cuda_probe.py:573-811): ``HipProbe`` (one-shot
route, arena create, query upload), ``HipDeviceArena`` (persistent bank with
host- and device-pointer route entries) and ``HipDeviceQueryPtr`` (owning
handle of a device query buffer).  The reference names ``CudaProbe``,
``CudaDeviceArena`` and ``CudaDeviceQueryPtr`` are aliases.

Behaviour kept from the reference: float32 C-contiguous inputs, row ids out
(uint64, UINT64_MAX for unfilled slots), ``RuntimeError(... code N)`` on a
nonzero return, ``ValueError`` for dim mismatch and topk > nodes, wall time
measured around the C call, device time from the ``warmup``-th query.
"""

from __future__ import annotations

import ctypes
import time
from pathlib import Path

import numpy as np

from . import _lib


def _fptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


class HipProbe:
    """Loaded MLA route library (mirrors CudaProbe, :573-626)."""

    def __init__(self, lib_path: Path | None = None):
        self.lib = _lib.load(lib_path)

    def upload_queries(self, queries: np.ndarray) -> "HipDeviceQueryPtr":
        queries = np.ascontiguousarray(queries, dtype=np.float32)
        handle = ctypes.c_void_p()
        rc = self.lib.grm_mla_cuda_upload_queries(
            _fptr(queries), ctypes.c_size_t(queries.size), ctypes.byref(handle))
        if rc != 0:
            raise RuntimeError(f"HIP query upload failed with code {rc}")
        return HipDeviceQueryPtr(self, handle, shape=queries.shape)

    def route_topk(self, rows: np.ndarray, queries: np.ndarray, *,
                   warmup: int, topk: int) -> tuple[np.ndarray, float, float]:
        rows = np.ascontiguousarray(rows, dtype=np.float32)
        queries = np.ascontiguousarray(queries, dtype=np.float32)
        nodes, dim = rows.shape
        query_count, query_dim = queries.shape
        if query_dim != dim:
            raise ValueError("query dim does not match rows")
        out = np.empty((query_count, topk), dtype=np.uint64)
        elapsed = ctypes.c_float(0.0)
        t0 = time.perf_counter_ns()
        rc = self.lib.grm_mla_cublas_route(
            _fptr(rows), _fptr(queries), nodes, dim, query_count, warmup, topk,
            _fptr(out), ctypes.byref(elapsed))
        wall_ms = (time.perf_counter_ns() - t0) / 1.0e6
        if rc != 0:
            raise RuntimeError(f"HIP MLA probe failed with code {rc}")
        return out, float(elapsed.value), wall_ms

    def create_arena(self, rows: np.ndarray) -> "HipDeviceArena":
        rows = np.ascontiguousarray(rows, dtype=np.float32)
        nodes, dim = rows.shape
        handle = ctypes.c_void_p()
        t0 = time.perf_counter_ns()
        rc = self.lib.grm_mla_cuda_arena_create(_fptr(rows), nodes, dim,
                                                ctypes.byref(handle))
        setup_wall_ms = (time.perf_counter_ns() - t0) / 1.0e6
        if rc != 0:
            raise RuntimeError(f"HIP MLA arena create failed with code {rc}")
        return HipDeviceArena(self, handle, nodes=nodes, dim=dim,
                              setup_wall_ms=setup_wall_ms)


class HipDeviceArena:
    """Persistent device MLA bank (mirrors CudaDeviceArena, :681-782)."""

    def __init__(self, probe: HipProbe, handle: ctypes.c_void_p, *, nodes: int,
                 dim: int, setup_wall_ms: float):
        self.probe = probe
        self.handle = handle
        self.nodes = nodes
        self.dim = dim
        self.setup_wall_ms = setup_wall_ms

    def close(self) -> None:
        if not self.handle:
            return
        rc = self.probe.lib.grm_mla_cuda_arena_destroy(self.handle)
        self.handle = ctypes.c_void_p()
        if rc != 0:
            raise RuntimeError(f"HIP MLA arena destroy failed with code {rc}")

    def __del__(self) -> None:
        if getattr(self, "handle", None):
            self.probe.lib.grm_mla_cuda_arena_destroy(self.handle)
            self.handle = ctypes.c_void_p()

    def route_topk(self, queries: np.ndarray, *, warmup: int,
                   topk: int) -> tuple[np.ndarray, float, float]:
        if not self.handle:
            raise RuntimeError("HIP MLA arena is closed")
        queries = np.ascontiguousarray(queries, dtype=np.float32)
        query_count, query_dim = queries.shape
        if query_dim != self.dim:
            raise ValueError("query dim does not match rows")
        if topk > self.nodes:
            raise ValueError("topk cannot exceed node count")
        out = np.empty((query_count, topk), dtype=np.uint64)
        elapsed = ctypes.c_float(0.0)
        t0 = time.perf_counter_ns()
        rc = self.probe.lib.grm_mla_cuda_arena_route(
            self.handle, _fptr(queries), query_count, self.dim, warmup, topk,
            _fptr(out), ctypes.byref(elapsed))
        wall_ms = (time.perf_counter_ns() - t0) / 1.0e6
        if rc != 0:
            raise RuntimeError(f"HIP MLA arena route failed with code {rc}")
        return out, float(elapsed.value), wall_ms

    def route_topk_device(self, device_queries: "HipDeviceQueryPtr", *,
                          warmup: int, topk: int
                          ) -> tuple[np.ndarray, float, float]:
        if not self.handle:
            raise RuntimeError("HIP MLA arena is closed")
        query_count, query_dim = device_queries.shape
        if query_dim != self.dim:
            raise ValueError("query dim does not match rows")
        if topk > self.nodes:
            raise ValueError("topk cannot exceed node count")
        out = np.empty((query_count, topk), dtype=np.uint64)
        elapsed = ctypes.c_float(0.0)
        t0 = time.perf_counter_ns()
        rc = self.probe.lib.grm_mla_cuda_arena_route_device(
            self.handle, device_queries.handle, query_count, self.dim, warmup,
            topk, _fptr(out), ctypes.byref(elapsed))
        wall_ms = (time.perf_counter_ns() - t0) / 1.0e6
        if rc != 0:
            raise RuntimeError(
                f"HIP MLA arena device route failed with code {rc}")
        return out, float(elapsed.value), wall_ms


class HipDeviceQueryPtr:
    """Owning handle of a device query buffer (mirrors CudaDeviceQueryPtr,
    :785-811).  ``.handle`` is the device pointer, ``.shape`` its shape."""

    def __init__(self, probe, handle: ctypes.c_void_p, *,
                 shape: tuple[int, ...]):
        self.probe = probe
        self.handle = handle
        self.shape = tuple(int(x) for x in shape)

    def close(self) -> None:
        if self.handle:
            self.probe.lib.grm_mla_cuda_free_device_ptr(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self) -> None:
        if getattr(self, "handle", None):
            self.probe.lib.grm_mla_cuda_free_device_ptr(self.handle)
            self.handle = ctypes.c_void_p()


# Reference names (scripts/grm_mla_cuda_probe.py) for drop-in callers.
CudaProbe = HipProbe
CudaDeviceArena = HipDeviceArena
CudaDeviceQueryPtr = HipDeviceQueryPtr
