"""HIP route sidecar: the drop-in for core/grm_cuda_router.py.

Same classes, functions, argument meaning and errors as the reference
module (core/grm_cuda_router.py:1-539), backed by libgrm_hip_router.so:

* ``CudaRouterUnavailable`` (:18) -- raised when the library cannot load;
* ``CudaRouteReceipt`` (:22-32) -- device/wall timings of a route call;
* ``validate_{gqa,mla}_route_bank`` (:35-57, :293-314) and the blake2b bank
  signatures (:60-75, :317-332);
* ``Cuda{GQA,MLA}RouteSidecar`` (:87-156, :344-405) with ``build()``,
  ``create_bank()``, ``close()``; ``build()`` loads the prebuilt library (the
  reference compiles CUDA with nvcc at this point, :101-125) and keeps the
  ``nvcc=`` keyword for signature compatibility;
* ``Cuda{GQA,MLA}RouteBank`` (:159-282, :408-539) with ``route_topk`` and
  ``route_topk_device``, row -> node id mapping and the out-of-range guard.

The ``Hip*`` names are the same objects.
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from . import _lib
from ._lib import HipRouterUnavailable
from .gqa_probe import HipProbe as HipGqaProbe
from .mla_probe import HipProbe as HipMlaProbe

CudaRouterUnavailable = HipRouterUnavailable


@dataclass(frozen=True)
class CudaRouteReceipt:
    device_route_ms_total: float
    device_route_ms_per_query: float
    route_wall_ms: float
    route_wall_ms_first: float
    route_wall_ms_min: float
    route_wall_ms_runs: tuple[float, ...]
    device_route_ms_runs: tuple[float, ...]
    measured_queries: int
    route_repeats: int


def validate_gqa_route_bank(keys: np.ndarray, node_ids: np.ndarray | None = None
                            ) -> tuple[np.ndarray, np.ndarray]:
    """Dense GQA bank of shape (nodes, kv_heads, key_tokens, head_dim)."""
    keys_np = np.ascontiguousarray(keys, dtype=np.float32)
    if keys_np.ndim != 4:
        raise ValueError(
            "GQA CUDA route bank must have shape "
            "(nodes, kv_heads, key_tokens, head_dim)")
    if any(int(dim) <= 0 for dim in keys_np.shape):
        raise ValueError("GQA CUDA route bank dimensions must be nonzero")
    if node_ids is None:
        ids_np = np.arange(keys_np.shape[0], dtype=np.uint64)
    else:
        ids_np = np.ascontiguousarray(node_ids, dtype=np.uint64).reshape(-1)
    if ids_np.shape[0] != keys_np.shape[0]:
        raise ValueError("node_ids length must match GQA route-bank nodes")
    return keys_np, ids_np


def _signature(arr: np.ndarray, ids: np.ndarray) -> str:
    digest = hashlib.blake2b(digest_size=16)
    digest.update(str(arr.shape).encode("ascii"))
    digest.update(arr.dtype.str.encode("ascii"))
    digest.update(memoryview(arr.view(np.uint8)))
    digest.update(str(ids.shape).encode("ascii"))
    digest.update(ids.dtype.str.encode("ascii"))
    digest.update(memoryview(ids.view(np.uint8)))
    return digest.hexdigest()


def gqa_route_bank_signature(keys: np.ndarray, node_ids: np.ndarray) -> str:
    keys_np, ids_np = validate_gqa_route_bank(keys, node_ids)
    return _signature(keys_np, ids_np)


def validate_mla_route_bank(rows: np.ndarray, node_ids: np.ndarray | None = None
                            ) -> tuple[np.ndarray, np.ndarray]:
    """Dense MLA bank of shape (nodes, dim): one centroid row per node."""
    rows_np = np.ascontiguousarray(rows, dtype=np.float32)
    if rows_np.ndim != 2:
        raise ValueError("MLA CUDA route bank must have shape (nodes, dim)")
    if any(int(dim) <= 0 for dim in rows_np.shape):
        raise ValueError("MLA CUDA route bank dimensions must be nonzero")
    if node_ids is None:
        ids_np = np.arange(rows_np.shape[0], dtype=np.uint64)
    else:
        ids_np = np.ascontiguousarray(node_ids, dtype=np.uint64).reshape(-1)
    if ids_np.shape[0] != rows_np.shape[0]:
        raise ValueError("node_ids length must match MLA route-bank nodes")
    return rows_np, ids_np


def mla_route_bank_signature(rows: np.ndarray, node_ids: np.ndarray) -> str:
    rows_np, ids_np = validate_mla_route_bank(rows, node_ids)
    return _signature(rows_np, ids_np)


def _load_or_unavailable(probe_cls, lib_path):
    try:
        return probe_cls(lib_path)
    except HipRouterUnavailable:
        raise
    except OSError as exc:  # pragma: no cover - loader errors vary
        raise HipRouterUnavailable(str(exc)) from exc


class _Sidecar:
    _probe_cls = None
    _bank_cls = None

    def __init__(self, lib_path: Path | None = None, *, build_temp=None):
        self._build_temp = build_temp
        self.lib_path = Path(lib_path) if lib_path else _lib.library_path()
        self._probe = _load_or_unavailable(self._probe_cls, self.lib_path)

    @classmethod
    def build(cls, build_dir: Path | None = None, *, nvcc: str = "nvcc"):
        """Load the prebuilt route library (``build_dir`` may name a directory
        holding libgrm_hip_router.so; ``nvcc`` is accepted and unused)."""
        del nvcc
        path = None
        if build_dir is not None:
            cand = Path(build_dir) / _lib.DEFAULT_LIB.name
            path = cand if cand.exists() else None
        return cls(path)

    def close(self) -> None:
        self._build_temp = None

    def __del__(self) -> None:
        self.close()


class _RouteBank:
    _kind = ""

    def __init__(self, arena, node_ids: np.ndarray, *, setup_wall_ms: float,
                 signature: object | None = None):
        self._arena = arena
        self.node_ids = np.ascontiguousarray(node_ids, dtype=np.uint64)
        self.setup_wall_ms = float(setup_wall_ms)
        self.signature = signature

    def close(self) -> None:
        if self._arena is not None:
            self._arena.close()
            self._arena = None

    def __del__(self) -> None:
        self.close()

    def _receipt_and_map(self, runs, query_count: int, warmup: int):
        topk_rows = runs[-1][0]
        if topk_rows is None:
            raise RuntimeError(f"HIP {self._kind} route did not run")
        # Unfilled slots are UINT64_MAX (fewer finite scores than topk);
        # the caller falls back exactly as with the reference sidecar.
        if np.any(topk_rows >= self.node_ids.shape[0]):
            raise RuntimeError(
                f"HIP {self._kind} route returned an out-of-range row ID")
        mapped = self.node_ids[topk_rows]
        walls = [float(r[2]) for r in runs]
        devs = [float(r[1]) for r in runs]
        measured = max(1, int(query_count) - int(warmup))
        receipt = CudaRouteReceipt(
            device_route_ms_total=devs[-1],
            device_route_ms_per_query=devs[-1] / measured,
            route_wall_ms=walls[-1],
            route_wall_ms_first=walls[0],
            route_wall_ms_min=float(np.min(walls)),
            route_wall_ms_runs=tuple(walls),
            device_route_ms_runs=tuple(devs),
            measured_queries=measured,
            route_repeats=len(runs),
        )
        return mapped, receipt

    def route_topk_device(self, device_queries, *, topk: int, warmup: int = 0,
                          route_repeats: int = 1):
        if self._arena is None:
            raise RuntimeError(f"HIP {self._kind} route bank is closed")
        if int(topk) <= 0:
            raise ValueError("topk must be positive")
        runs = [self._arena.route_topk_device(device_queries,
                                              warmup=int(warmup),
                                              topk=int(topk))
                for _ in range(max(1, int(route_repeats)))]
        return self._receipt_and_map(runs, device_queries.shape[0], warmup)


class CudaGQARouteBank(_RouteBank):
    """Device-resident GQA bank (mirrors core/grm_cuda_router.py:159-282)."""

    _kind = "GQA"

    def route_topk(self, queries: np.ndarray, *, topk: int, warmup: int = 0,
                   route_repeats: int = 1):
        if self._arena is None:
            raise RuntimeError("HIP GQA route bank is closed")
        queries_np = np.ascontiguousarray(queries, dtype=np.float32)
        if queries_np.ndim == 3:
            queries_np = queries_np[None, ...]
        if queries_np.ndim != 4:
            raise ValueError(
                "GQA CUDA queries must have shape "
                "(queries, heads, tokens, dim) or (heads, tokens, dim)")
        if int(topk) <= 0:
            raise ValueError("topk must be positive")
        runs = [self._arena.route_topk(queries_np, warmup=int(warmup),
                                       topk=int(topk))
                for _ in range(max(1, int(route_repeats)))]
        return self._receipt_and_map(runs, queries_np.shape[0], warmup)


class CudaMLARouteBank(_RouteBank):
    """Device-resident MLA bank (mirrors core/grm_cuda_router.py:408-539)."""

    _kind = "MLA"

    def route_topk(self, queries: np.ndarray, *, topk: int, warmup: int = 0,
                   route_repeats: int = 1):
        if self._arena is None:
            raise RuntimeError("HIP MLA route bank is closed")
        queries_np = np.ascontiguousarray(queries, dtype=np.float32)
        if queries_np.ndim == 1:
            queries_np = queries_np[None, ...]
        if queries_np.ndim != 2:
            raise ValueError(
                "MLA CUDA queries must have shape (queries, dim) or (dim,)")
        if int(topk) <= 0:
            raise ValueError("topk must be positive")
        runs = [self._arena.route_topk(queries_np, warmup=int(warmup),
                                       topk=int(topk))
                for _ in range(max(1, int(route_repeats)))]
        return self._receipt_and_map(runs, queries_np.shape[0], warmup)


class CudaGQARouteSidecar(_Sidecar):
    """Load the HIP GQA route library (mirrors :87-156)."""

    _probe_cls = HipGqaProbe

    def create_bank(self, keys: np.ndarray, node_ids: np.ndarray | None = None,
                    *, signature: object | None = None) -> CudaGQARouteBank:
        keys_np, ids_np = validate_gqa_route_bank(keys, node_ids)
        if signature is None:
            signature = _signature(keys_np, ids_np)
        arena = self._probe.create_arena(keys_np)
        return CudaGQARouteBank(arena, ids_np,
                                setup_wall_ms=float(arena.setup_wall_ms),
                                signature=signature)


class CudaMLARouteSidecar(_Sidecar):
    """Load the HIP MLA route library (mirrors :344-405)."""

    _probe_cls = HipMlaProbe

    def create_bank(self, rows: np.ndarray, node_ids: np.ndarray | None = None
                    ) -> CudaMLARouteBank:
        rows_np, ids_np = validate_mla_route_bank(rows, node_ids)
        signature = _signature(rows_np, ids_np)
        arena = self._probe.create_arena(rows_np)
        return CudaMLARouteBank(arena, ids_np,
                                setup_wall_ms=float(arena.setup_wall_ms),
                                signature=signature)


HipRouteReceipt = CudaRouteReceipt
HipGQARouteSidecar = CudaGQARouteSidecar
HipGQARouteBank = CudaGQARouteBank
HipMLARouteSidecar = CudaMLARouteSidecar
HipMLARouteBank = CudaMLARouteBank

__all__ = [
    "CudaRouterUnavailable", "HipRouterUnavailable", "CudaRouteReceipt",
    "HipRouteReceipt", "validate_gqa_route_bank", "gqa_route_bank_signature",
    "validate_mla_route_bank", "mla_route_bank_signature",
    "CudaGQARouteSidecar", "CudaGQARouteBank", "CudaMLARouteSidecar",
    "CudaMLARouteBank", "HipGQARouteSidecar", "HipGQARouteBank",
    "HipMLARouteSidecar", "HipMLARouteBank",
]
