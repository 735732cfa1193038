"""MI355X (gfx950) GRM graft router.

The route hot path of GraftRepository -- score every stored graft's route key
against a query and return the top-k node ids -- as a HIP shared library
(libgrm_hip_router.so) behind the reference sidecar's C ABI and Python
surface.

* ``grm_hip_router`` / ``grm_cuda_router``: drop-in for core/grm_cuda_router.py
* ``mla_probe`` / ``gqa_probe``: drop-in for the probes' ctypes layers
* ``node_bank``: ids + scores, bf16/fp16/int8 banks, ragged CSR, append/evict
* ``bank_bridge``: epoch-gated banks that follow an arena's grafts with
  evictions and appends instead of full rebuilds
* ``workloads``: seeded synthetic route workloads
"""

from ._lib import HipRouterUnavailable, library_path, load, runtime_info
from .node_bank import GqaNodeBank, MlaNodeBank, RouteResult
from .bank_bridge import GqaRouteBankBridge, MlaRouteBankBridge

__all__ = ["HipRouterUnavailable", "library_path", "load", "runtime_info",
           "GqaNodeBank", "MlaNodeBank", "RouteResult", "GqaRouteBankBridge",
           "MlaRouteBankBridge"]
