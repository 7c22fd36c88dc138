"""In-tree build of libmednext_hip.so (hipcc, gfx950 only).

Every call recompiles: the sources are compiled to objects in parallel and linked
into ``_lib/libmednext_hip.so`` next to this file, replaced atomically. The
library links against ``libamdhip64.so.7``; imported after ``torch`` it binds to
the HIP runtime PyTorch already loaded (same SONAME), so device pointers and
streams are shared with PyTorch.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
CSRC_DIR = PACKAGE_DIR.parent / "csrc"
INCLUDE_DIR = PACKAGE_DIR.parent.parent / "include"
LIB_DIR = PACKAGE_DIR / "_lib"
LIB_NAME = "libmednext_hip.so"
LIB_PATH = LIB_DIR / LIB_NAME

ARCH = "gfx950"
SOURCES = (
    "capi.hip", "depthwise.hip", "depthwise_mfma.hip", "depthwise_volume.hip", "groupnorm.hip", "grn.hip",
    "pointwise.hip", "upjoin.hip",
)

# Packed FP32 VALU instructions are disabled for all device code: some of
# their forms have produced silent wrong results on the target machines.
HIPCC_FLAGS = (
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
)


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    candidate = Path(rocm) / "bin" / "hipcc"
    if candidate.exists():
        return str(candidate)
    found = shutil.which("hipcc")
    if found is None:
        raise RuntimeError("hipcc not found; set ROCM_PATH")
    return found


def _compile(source: Path, obj: Path) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{INCLUDE_DIR}", "-c", str(source), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{' '.join(cmd)}\n{result.stderr}")


def build(verbose: bool = False) -> Path:
    """Compile every HIP source for gfx950 and link the C-ABI shared library."""
    sources = [CSRC_DIR / name for name in SOURCES if (CSRC_DIR / name).exists()]
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC_DIR}")
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    with tempfile.TemporaryDirectory(prefix="mednext_build_") as tmp:
        objs = [Path(tmp) / (src.stem + ".o") for src in sources]
        workers = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
        with ThreadPoolExecutor(max_workers=workers) as pool:
            list(pool.map(_compile, sources, objs))
        staged = Path(tmp) / LIB_NAME
        cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(staged)]
        result = subprocess.run(cmd, capture_output=True, text=True)
        if result.returncode != 0:
            raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{result.stderr}")
        target_tmp = LIB_DIR / (LIB_NAME + ".tmp")
        shutil.copyfile(staged, target_tmp)
        os.replace(target_tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
