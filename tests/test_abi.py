"""The C-ABI library loads and exports exactly what include/grm_hip_router.h
declares (CPU only: no compute calls)."""

import re
import subprocess
from pathlib import Path

import pytest

import graftrepository_amd as g
from graftrepository_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "grm_hip_router.h"

# The reference sidecar's exported names (scripts/grm_mla_cuda_probe.py,
# scripts/grm_gqa_cuda_probe.py), which must all be present unchanged.
REFERENCE_SYMBOLS = {
    "grm_mla_cuda_arena_create", "grm_mla_cuda_arena_route",
    "grm_mla_cuda_arena_route_device", "grm_mla_cuda_upload_queries",
    "grm_mla_cuda_free_device_ptr", "grm_mla_cuda_arena_destroy",
    "grm_mla_cublas_route", "grm_gqa_cuda_arena_create",
    "grm_gqa_cuda_arena_route", "grm_gqa_cuda_arena_route_device",
    "grm_gqa_cuda_upload_queries", "grm_gqa_cuda_free_device_ptr",
    "grm_gqa_cuda_arena_destroy", "grm_gqa_cublas_route",
    # the CPU store's route calls (cpp/grm_runtime_c.h:176-181, 381-436, 499)
    "grm_store_set_route", "grm_store_set_route_multi", "grm_store_set_route_list",
    "grm_store_clear_route", "grm_store_set_route_metadata", "grm_store_route",
    "grm_store_route_filtered", "grm_store_route_gqa", "grm_store_last_error",
}


def header_functions() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(grm_\w+)\s*\(", text))


def exported_symbols() -> set[str]:
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.library_path())],
                         capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines()
            if " T " in line and line.split()[-1].startswith("grm_")}


def test_library_is_built_and_loads():
    lib = g.load()
    assert lib is not None


def test_header_and_exports_agree():
    declared = header_functions()
    assert REFERENCE_SYMBOLS <= declared
    assert exported_symbols() == declared
    assert set(_lib.SIGNATURES) == declared


def test_every_declared_symbol_resolves_through_ctypes():
    lib = g.load()
    for name in header_functions():
        assert getattr(lib, name) is not None


def test_missing_library_raises_unavailable(tmp_path, monkeypatch):
    monkeypatch.setenv("GRM_HIP_ROUTER_LIB", str(tmp_path / "nope.so"))
    with pytest.raises(g.HipRouterUnavailable):
        _lib.load()
    from graftrepository_amd.grm_hip_router import (CudaMLARouteSidecar,
                                                    CudaRouterUnavailable)
    with pytest.raises(CudaRouterUnavailable):
        CudaMLARouteSidecar.build()


def test_library_carries_a_gfx950_code_object():
    # The offload bundle of the library built here names its target triple.
    blob = _lib.library_path().read_bytes()
    assert b"amdgcn-amd-amdhsa--gfx950" in blob
