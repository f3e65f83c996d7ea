"""Compile libayaka_hip.so for gfx950 with hipcc, in-tree.

The library is the C-ABI of the HIP kernels (``include/ayaka_hip.h``); Python
reaches it through :mod:`ctypes`, so nothing here links against torch.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

__all__ = ["FLAGS", "LIB_PATH", "build_library", "hipcc_command"]

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_DIR = PACKAGE_DIR.parent
SOURCES = ("api.hip", "paged_attention.hip", "paged_attention_mfma.hip", "paged_prefill.hip", "kv_cache.hip",
           "paged_attention_f32.hip", "split_model.cpp", "kv_reach.hip")
LIB_PATH = PACKAGE_DIR / "lib" / "libayaka_hip.so"
ARCH = "gfx950"


def _hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found: the HIP library cannot be built")
    return found


FLAGS = (
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    # Packed fp32 VALU ops are kept out of every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
)


def hipcc_command(source: Path, output: Path) -> list[str]:
    """The hipcc line that compiles one source into an object."""
    csrc = PACKAGE_DIR / "csrc"
    return [_hipcc(), *FLAGS, f"-I{REPO_DIR / 'include'}", f"-I{csrc}", "-c", str(source), "-o", str(output)]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    result = subprocess.run(cmd, capture_output=True, text=True, check=False)
    if result.returncode != 0:
        sys.stderr.write(result.stdout + result.stderr)
        raise RuntimeError(f"hipcc failed with exit code {result.returncode}: {' '.join(cmd)}")


def build_library(*, verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every HIP source (in parallel) and link ``ayaka_amd/lib/libayaka_hip.so``."""
    out_dir = LIB_PATH.parent
    obj_dir = out_dir / "obj"
    obj_dir.mkdir(parents=True, exist_ok=True)
    csrc = PACKAGE_DIR / "csrc"
    objects = [obj_dir / (Path(name).stem + ".o") for name in SOURCES]
    workers = jobs or min(len(SOURCES), os.cpu_count() or 1, 16)
    with ThreadPoolExecutor(max_workers=workers) as pool:
        for future in [pool.submit(_run, hipcc_command(csrc / name, obj), verbose)
                       for name, obj in zip(SOURCES, objects)]:
            future.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)], verbose)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build_library(verbose=True))
