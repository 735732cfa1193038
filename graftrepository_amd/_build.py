"""Build libgrm_hip_router.so (gfx950) in-tree with hipcc.

Every ``csrc/*.hip`` file is compiled to an object in parallel and linked
into ``graftrepository_amd/libgrm_hip_router.so``.  Flags:

* ``--offload-arch=gfx950`` only (MI355X);
* ``-ffp-contract=off``: the route laws' fp64 expressions must round exactly
  as written (explicit ``fma`` is used where a fused product is exact);
* ``-Xclang -target-feature -Xclang -packed-fp32-ops``: no packed fp32 VALU
  instructions are generated.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
LIB_NAME = "libgrm_hip_router.so"
LIB_PATH = PKG / LIB_NAME
OBJ_DIR = PKG / "_build"
ARCH = os.environ.get("GRM_HIP_ARCH", "gfx950")

COMMON_FLAGS = [
    "-std=c++17", "-O3", f"--offload-arch={ARCH}", "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
    f"-I{INCLUDE}", f"-I{CSRC}",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc",
                 shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise FileNotFoundError("hipcc not found")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


# Per-source flags.  mla_route.hip: MFMA accumulators in VGPRs (the ring
# screen keeps its query fragments in AGPRs and reduces the accumulators
# with VALU instructions, which then need no AGPR-to-VGPR copies).
SOURCE_FLAGS = {
    "mla_route.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def _compile(src: Path) -> Path:
    obj = OBJ_DIR / (src.stem + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, *SOURCE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every source and link the shared library (always rebuilds)."""
    OBJ_DIR.mkdir(exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    # -z defs: a symbol left undefined fails the link (a kernel template
    # whose host-side instantiation was dropped would otherwise surface
    # only when the library is loaded)
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-z,defs",
           *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    tmp.replace(LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
