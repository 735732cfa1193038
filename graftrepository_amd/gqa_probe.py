"""Drop-in for the GQA sidecar probe's ctypes layer
(scripts/grm_gqa_cuda_probe.py:632-911): ``HipProbe`` binds the shared
layer of ``probe`` to the GQA entry points.  Banks are the reference's
dense zero-padded ``[nodes, kv_heads, key_tokens, head_dim]`` fp32 arrays,
queries ``[Q, heads, tokens, head_dim]``; the library keeps the bank as a
CSR bank (a padding token scores |0| = 0 and never changes a maximum).
Ragged, bf16/fp16/int8 and mutable banks use ``node_bank.GqaNodeBank``.
The reference's names are aliases."""

from __future__ import annotations

from .probe import GQA, DeviceQueryPtr, ProbeArena, RouteProbe


class HipProbe(RouteProbe):
    dialect = GQA


HipDeviceArena = ProbeArena
HipDeviceQueryPtr = DeviceQueryPtr
CudaProbe = HipProbe
CudaDeviceArena = ProbeArena
CudaDeviceQueryPtr = DeviceQueryPtr
