"""Compile libayaka_hip.so for gfx950 with hipcc, in-tree.

The library is the C-ABI of the HIP kernels (``include/ayaka_hip.h``); Python
reaches it through :mod:`ctypes`, so nothing here links against torch.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

__all__ = ["LIB_PATH", "build_library", "hipcc_command"]

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_DIR = PACKAGE_DIR.parent
SOURCES = ("api.hip", "paged_attention.hip", "kv_cache.hip")
LIB_PATH = PACKAGE_DIR / "lib" / "libayaka_hip.so"
ARCH = "gfx950"


def _hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found: the HIP library cannot be built")
    return found


def hipcc_command(output: Path = LIB_PATH, extra: tuple[str, ...] = ()) -> list[str]:
    """The one hipcc line that builds the shared library."""
    csrc = PACKAGE_DIR / "csrc"
    return [
        _hipcc(),
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-Wall",
        # Packed fp32 VALU ops are kept out of every kernel.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        f"-I{REPO_DIR / 'include'}",
        f"-I{csrc}",
        *extra,
        *(str(csrc / name) for name in SOURCES),
        "-o",
        str(output),
    ]


def build_library(*, verbose: bool = False) -> Path:
    """Compile every HIP source into ``ayaka_amd/lib/libayaka_hip.so`` and return its path."""
    LIB_PATH.parent.mkdir(parents=True, exist_ok=True)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = hipcc_command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    env = dict(os.environ)
    result = subprocess.run(cmd, capture_output=True, text=True, env=env, check=False)
    if result.returncode != 0:
        sys.stderr.write(result.stdout + result.stderr)
        raise RuntimeError(f"hipcc failed with exit code {result.returncode}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build_library(verbose=True))
