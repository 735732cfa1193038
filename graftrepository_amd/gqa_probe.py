"""Host binding of the GQA route library, mirroring the reference probe's
ctypes layer (scripts/grm_gqa_cuda_probe.py:632-911): ``HipProbe`` (one-shot
route, arena create, query upload), ``HipDeviceArena`` (persistent dense
bank with host- and device-pointer route entries) and ``HipDeviceQueryPtr``.
The reference names ``CudaProbe``, ``CudaDeviceArena`` and
``CudaDeviceQueryPtr`` are aliases.

Banks handed to this layer are the reference's dense zero-padded
[nodes, kv_heads, key_tokens, head_dim] fp32 arrays; the library stores them
as a CSR bank (padding tokens score |0| = 0 and never change a maximum).
Ragged, bf16/fp16/int8 and mutable banks use ``node_bank.GqaNodeBank``.
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
    """Loaded GQA route library (mirrors CudaProbe, :632-762)."""

    def __init__(self, lib_path: Path | None = None):
        self.lib = _lib.load(lib_path)

    def upload_queries(self, queries: np.ndarray) -> "HipDeviceQueryPtr":
        queries = np.ascontiguousarray(queries, dtype=np.float32)
        handle = ctypes.c_void_p()
        rc = self.lib.grm_gqa_cuda_upload_queries(
            _fptr(queries), ctypes.c_size_t(queries.size), ctypes.byref(handle))
        if rc != 0:
            raise RuntimeError(f"HIP query upload failed with code {rc}")
        return HipDeviceQueryPtr(self, handle, shape=queries.shape)

    def route_topk(self, keys: np.ndarray, queries: np.ndarray, *,
                   warmup: int, topk: int) -> tuple[np.ndarray, float, float]:
        keys = np.ascontiguousarray(keys, dtype=np.float32)
        queries = np.ascontiguousarray(queries, dtype=np.float32)
        nodes, kv_heads, key_tokens, head_dim = keys.shape
        query_count, query_heads, query_tokens, query_dim = queries.shape
        if query_dim != head_dim:
            raise ValueError("query head_dim does not match keys")
        out = np.empty((query_count, topk), dtype=np.uint64)
        elapsed = ctypes.c_float(0.0)
        t0 = time.perf_counter_ns()
        rc = self.lib.grm_gqa_cublas_route(
            _fptr(keys), _fptr(queries), nodes, kv_heads, key_tokens,
            query_count, query_heads, query_tokens, head_dim, warmup, topk,
            _fptr(out), ctypes.byref(elapsed))
        wall_ms = (time.perf_counter_ns() - t0) / 1.0e6
        if rc != 0:
            raise RuntimeError(f"HIP GQA probe failed with code {rc}")
        return out, float(elapsed.value), wall_ms

    def create_arena(self, keys: np.ndarray) -> "HipDeviceArena":
        keys = np.ascontiguousarray(keys, dtype=np.float32)
        nodes, kv_heads, key_tokens, head_dim = keys.shape
        handle = ctypes.c_void_p()
        t0 = time.perf_counter_ns()
        rc = self.lib.grm_gqa_cuda_arena_create(
            _fptr(keys), nodes, kv_heads, key_tokens, head_dim,
            ctypes.byref(handle))
        setup_wall_ms = (time.perf_counter_ns() - t0) / 1.0e6
        if rc != 0:
            raise RuntimeError(f"HIP arena create failed with code {rc}")
        return HipDeviceArena(self, handle, nodes=nodes, kv_heads=kv_heads,
                              key_tokens=key_tokens, head_dim=head_dim,
                              setup_wall_ms=setup_wall_ms)


class HipDeviceArena:
    """Persistent device GQA bank (mirrors CudaDeviceArena, :765-880)."""

    def __init__(self, probe: HipProbe, handle: ctypes.c_void_p, *, nodes: int,
                 kv_heads: int, key_tokens: int, head_dim: int,
                 setup_wall_ms: float):
        self.probe = probe
        self.handle = handle
        self.nodes = nodes
        self.kv_heads = kv_heads
        self.key_tokens = key_tokens
        self.head_dim = head_dim
        self.setup_wall_ms = setup_wall_ms

    def close(self) -> None:
        if not self.handle:
            return
        rc = self.probe.lib.grm_gqa_cuda_arena_destroy(self.handle)
        self.handle = ctypes.c_void_p()
        if rc != 0:
            raise RuntimeError(f"HIP arena destroy failed with code {rc}")

    def __del__(self) -> None:
        if getattr(self, "handle", None):
            self.probe.lib.grm_gqa_cuda_arena_destroy(self.handle)
            self.handle = ctypes.c_void_p()

    def route_topk(self, queries: np.ndarray, *, warmup: int,
                   topk: int) -> tuple[np.ndarray, float, float]:
        if not self.handle:
            raise RuntimeError("HIP arena is closed")
        queries = np.ascontiguousarray(queries, dtype=np.float32)
        query_count, query_heads, query_tokens, query_dim = queries.shape
        if query_dim != self.head_dim:
            raise ValueError("query head_dim does not match keys")
        if topk > self.nodes:
            raise ValueError("topk cannot exceed node count")
        out = np.empty((query_count, topk), dtype=np.uint64)
        elapsed = ctypes.c_float(0.0)
        t0 = time.perf_counter_ns()
        rc = self.probe.lib.grm_gqa_cuda_arena_route(
            self.handle, _fptr(queries), query_count, query_heads,
            query_tokens, warmup, topk, _fptr(out), ctypes.byref(elapsed))
        wall_ms = (time.perf_counter_ns() - t0) / 1.0e6
        if rc != 0:
            raise RuntimeError(f"HIP arena route failed with code {rc}")
        return out, float(elapsed.value), wall_ms

    def route_topk_device(self, device_queries: "HipDeviceQueryPtr", *,
                          warmup: int, topk: int
                          ) -> tuple[np.ndarray, float, float]:
        if not self.handle:
            raise RuntimeError("HIP arena is closed")
        query_count, query_heads, query_tokens, query_dim = device_queries.shape
        if query_dim != self.head_dim:
            raise ValueError("query head_dim does not match keys")
        if topk > self.nodes:
            raise ValueError("topk cannot exceed node count")
        out = np.empty((query_count, topk), dtype=np.uint64)
        elapsed = ctypes.c_float(0.0)
        t0 = time.perf_counter_ns()
        rc = self.probe.lib.grm_gqa_cuda_arena_route_device(
            self.handle, device_queries.handle, query_count, query_heads,
            query_tokens, warmup, topk, _fptr(out), ctypes.byref(elapsed))
        wall_ms = (time.perf_counter_ns() - t0) / 1.0e6
        if rc != 0:
            raise RuntimeError(
                f"HIP arena device route failed with code {rc}")
        return out, float(elapsed.value), wall_ms


class HipDeviceQueryPtr:
    """Owning handle of a device query buffer (mirrors CudaDeviceQueryPtr,
    :883-911)."""

    def __init__(self, probe, handle: ctypes.c_void_p, *,
                 shape: tuple[int, ...]):
        self.probe = probe
        self.handle = handle
        self.shape = tuple(int(x) for x in shape)

    def close(self) -> None:
        if self.handle:
            self.probe.lib.grm_gqa_cuda_free_device_ptr(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self) -> None:
        if getattr(self, "handle", None):
            self.probe.lib.grm_gqa_cuda_free_device_ptr(self.handle)
            self.handle = ctypes.c_void_p()


CudaProbe = HipProbe
CudaDeviceArena = HipDeviceArena
CudaDeviceQueryPtr = HipDeviceQueryPtr
