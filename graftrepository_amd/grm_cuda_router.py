"""Import-path alias of :mod:`graftrepository_amd.grm_hip_router` so callers
of core/grm_cuda_router.py can switch by changing the package prefix only."""

from .grm_hip_router import *  # noqa: F401,F403
from .grm_hip_router import __all__  # noqa: F401
