"""ctypes binding of libgrm_hip_router.so (the gfx950 route library).

The library is loaded from ``GRM_HIP_ROUTER_LIB`` when set, else from the
package directory (built in-tree by ``graftrepository_amd._build``).  A
missing or unloadable library raises :class:`HipRouterUnavailable`; there is
no CPU fallback on this path.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

PKG = Path(__file__).resolve().parent
DEFAULT_LIB = PKG / "libgrm_hip_router.so"

DTYPE_F32, DTYPE_BF16, DTYPE_F16, DTYPE_I8 = 0, 1, 2, 3
DTYPE_CODES = {"f32": DTYPE_F32, "float32": DTYPE_F32, "bf16": DTYPE_BF16,
               "bfloat16": DTYPE_BF16, "f16": DTYPE_F16, "float16": DTYPE_F16,
               "i8": DTYPE_I8, "int8": DTYPE_I8}


class HipRouterUnavailable(RuntimeError):
    """The route library cannot be loaded (mirrors CudaRouterUnavailable,
    core/grm_cuda_router.py:18-19)."""


vp, u64, i32, f32p = (ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int,
                      ctypes.POINTER(ctypes.c_float))
u64p = ctypes.POINTER(ctypes.c_uint64)
sz = ctypes.c_size_t

# symbol -> (restype, argtypes); declared in include/grm_hip_router.h
SIGNATURES = {
    # reference MLA ABI (scripts/grm_mla_cuda_probe.py:575-626)
    "grm_mla_cuda_arena_create": (i32, [vp, i32, i32, ctypes.POINTER(vp)]),
    "grm_mla_cuda_arena_route": (i32, [vp, vp, i32, i32, i32, i32, vp, vp]),
    "grm_mla_cuda_arena_route_device": (i32, [vp, vp, i32, i32, i32, i32, vp,
                                              vp]),
    "grm_mla_cuda_upload_queries": (i32, [vp, sz, ctypes.POINTER(vp)]),
    "grm_mla_cuda_free_device_ptr": (i32, [vp]),
    "grm_mla_cuda_arena_destroy": (i32, [vp]),
    "grm_mla_cublas_route": (i32, [vp, vp, i32, i32, i32, i32, i32, vp, vp]),
    # reference GQA ABI (scripts/grm_gqa_cuda_probe.py:634-697)
    "grm_gqa_cuda_arena_create": (i32, [vp, i32, i32, i32, i32,
                                        ctypes.POINTER(vp)]),
    "grm_gqa_cuda_arena_route": (i32, [vp, vp, i32, i32, i32, i32, i32, vp,
                                       vp]),
    "grm_gqa_cuda_arena_route_device": (i32, [vp, vp, i32, i32, i32, i32, i32,
                                              vp, vp]),
    "grm_gqa_cuda_upload_queries": (i32, [vp, sz, ctypes.POINTER(vp)]),
    "grm_gqa_cuda_free_device_ptr": (i32, [vp]),
    "grm_gqa_cuda_arena_destroy": (i32, [vp]),
    "grm_gqa_cublas_route": (i32, [vp, vp, i32, i32, i32, i32, i32, i32, i32,
                                   i32, i32, vp, vp]),
    # extensions
    "grm_hip_last_error": (ctypes.c_char_p, []),
    "grm_hip_runtime_info": (i32, [ctypes.c_char_p, sz]),
    "grm_mla_hip_bank_create": (i32, [vp, i32, u64, i32, vp, u64,
                                      ctypes.POINTER(vp)]),
    "grm_mla_hip_route": (i32, [vp, vp, i32, i32, i32, i32, i32, i32, vp, vp,
                                vp]),
    "grm_mla_hip_route_noalloc": (i32, [vp, vp, i32, i32, i32, i32, vp, vp]),
    "grm_mla_hip_append": (i32, [vp, vp, i32, u64, vp, vp]),
    "grm_mla_hip_evict": (i32, [vp, vp, u64, vp]),
    "grm_mla_hip_sync": (i32, [vp]),
    "grm_mla_hip_bank_info": (i32, [vp, vp]),
    "grm_mla_hip_route_stats": (i32, [vp, vp]),
    "grm_mla_hip_screen_ms": (i32, [vp, vp]),
    "grm_mla_hip_probe_screen": (i32, [vp, vp, i32, i32, vp, vp, vp]),
    "grm_mla_hip_latent_query": (i32, [vp, vp, i32, u64, u64, i32, vp]),
    "grm_mla_hip_route_latent": (i32, [vp, vp, i32, u64, u64, i32, vp, vp, vp]),
    "grm_mla_hip_set_filter_bits": (i32, [vp, vp, vp, u64]),
    "grm_mla_hip_route_filtered": (i32, [vp, vp, i32, i32, i32, u64, ctypes.c_uint32, vp, vp,
                                         vp]),
    "grm_mla_hip_score_nodes": (i32, [vp, vp, i32, vp, u64, vp]),
    "grm_gqa_hip_bank_create": (i32, [vp, i32, vp, i32, i32, vp, u64, i32, i32,
                                      vp, u64, u64, ctypes.POINTER(vp)]),
    "grm_gqa_hip_route": (i32, [vp, vp, i32, i32, i32, i32, i32, i32, i32, vp,
                                vp, vp]),
    "grm_gqa_hip_append": (i32, [vp, vp, vp, vp, u64, vp, vp]),
    "grm_gqa_hip_evict": (i32, [vp, vp, u64, vp]),
    "grm_gqa_hip_compact": (i32, [vp]),
    "grm_gqa_hip_sync": (i32, [vp]),
    "grm_gqa_hip_bank_info": (i32, [vp, vp]),
    "grm_gqa_hip_route_stats": (i32, [vp, vp]),
    "grm_gqa_hip_probe_screen": (i32, [vp, vp, i32, i32, i32, vp, vp, vp, vp]),
    "grm_gqa_hip_set_filter_bits": (i32, [vp, vp, vp, u64]),
    "grm_gqa_hip_route_filtered": (i32, [vp, vp, i32, i32, i32, i32, i32, u64, ctypes.c_uint32,
                                         vp, vp, vp]),
    "grm_gqa_hip_score_nodes": (i32, [vp, vp, i32, i32, i32, vp, u64, vp]),
    # the store's route calls over a device bank (cpp/grm_runtime_c.h:176-181,
    # 381-436, 499) and their extensions
    "grm_hip_store_create_mla": (i32, [i32, u64, i32, ctypes.POINTER(vp)]),
    "grm_hip_store_create_gqa": (i32, [i32, i32, u64, u64, ctypes.POINTER(vp)]),
    "grm_hip_store_destroy": (None, [vp]),
    "grm_store_set_route": (i32, [vp, u64, vp, u64, ctypes.c_char_p]),
    "grm_store_set_route_multi": (i32, [vp, u64, vp, u64, u64, ctypes.c_char_p]),
    "grm_store_set_route_list": (i32, [vp, u64, vp, u64, vp, u64, ctypes.c_char_p]),
    "grm_store_clear_route": (i32, [vp, u64]),
    "grm_store_set_route_metadata": (i32, [vp, u64] + [ctypes.c_char_p] * 4),
    "grm_store_route": (i32, [vp, vp, u64, ctypes.c_char_p, u64, vp, u64, vp]),
    "grm_store_route_filtered": (i32, [vp, vp, u64] + [ctypes.c_char_p] * 5
                                 + [u64, vp, u64, vp]),
    "grm_store_route_gqa": (i32, [vp, vp, u64, u64, u64] + [ctypes.c_char_p] * 5
                            + [u64, vp, u64, vp]),
    "grm_store_last_error": (ctypes.c_char_p, [vp]),
    "grm_hip_store_set_routes": (i32, [vp, u64, vp, vp, vp, vp, vp]),
    "grm_hip_store_route_scored": (i32, [vp, vp, u64, u64] + [ctypes.c_char_p] * 5
                                   + [u64, vp, vp, u64, vp]),
    "grm_hip_store_info": (i32, [vp, vp]),
    "grm_hip_payload_dequant": (i32, [vp, vp, u64, ctypes.c_uint32, vp, vp]),
    "grm_hip_payload_upload": (i32, [vp, vp, u64, ctypes.c_uint32, vp, vp]),
    "grm_hip_device_alloc": (i32, [u64, ctypes.POINTER(vp)]),
    "grm_hip_device_free": (i32, [vp]),
    "grm_hip_copy_to_host": (i32, [vp, vp, u64]),
    "grm_hip_copy_to_device": (i32, [vp, vp, u64]),
    "grm_hip_synth_int8_rows": (i32, [u64, u64, u64, i32, vp, i32, vp, vp]),
}

_libs: dict[str, ctypes.CDLL] = {}


def library_path() -> Path:
    env = os.environ.get("GRM_HIP_ROUTER_LIB")
    return Path(env) if env else DEFAULT_LIB


def load(path: str | Path | None = None) -> ctypes.CDLL:
    """Load the route library once per path; raise HipRouterUnavailable if
    it is absent or does not export the declared symbols.

    The library binds to the HIP runtime the process has mapped under the
    soname libamdhip64.so.7 (ROCm's, unless another copy is mapped first).
    PyTorch wheels bundle their own copy of that runtime, opened under a
    different file name, so a process that imports torch after this load
    maps a second HIP and HSA runtime beside the first, and torch may then
    find no device.  A process that uses both imports torch first: the
    library then binds to torch's copy and the two share one runtime."""
    path = Path(path) if path is not None else library_path()
    key = str(path.resolve()) if path.exists() else str(path)
    if key in _libs:
        return _libs[key]
    if not path.exists():
        raise HipRouterUnavailable(
            f"{path} is not built; run graftrepository_amd._build.build()")
    try:
        lib = ctypes.CDLL(str(path))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
    except (OSError, AttributeError) as exc:
        raise HipRouterUnavailable(str(exc)) from exc
    _libs[key] = lib
    return lib


def last_error() -> str:
    msg = load().grm_hip_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


def check(rc: int, what: str) -> None:
    if rc != 0:
        detail = last_error()
        raise RuntimeError(f"{what} failed with code {rc}"
                           + (f": {detail}" if detail else ""))


def runtime_info() -> str:
    buf = ctypes.create_string_buffer(512)
    check(load().grm_hip_runtime_info(buf, len(buf)), "runtime_info")
    return buf.value.decode()
