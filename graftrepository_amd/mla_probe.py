"""Drop-in for the MLA sidecar probe's ctypes layer
(scripts/grm_mla_cuda_probe.py:573-811): ``HipProbe`` binds the shared
layer of ``probe`` to the MLA entry points (banks ``[nodes, dim]``,
queries ``[Q, dim]``).  The reference's names are aliases."""

from __future__ import annotations

from .probe import MLA, DeviceQueryPtr, ProbeArena, RouteProbe


class HipProbe(RouteProbe):
    dialect = MLA


HipDeviceArena = ProbeArena
HipDeviceQueryPtr = DeviceQueryPtr
CudaProbe = HipProbe
CudaDeviceArena = ProbeArena
CudaDeviceQueryPtr = DeviceQueryPtr
