"""Build the HIP library `libbpt_amd.so` for gfx950 from `csrc/`, in-tree, with hipcc.

Every `.hip` file under `csrc/` is compiled to an object (in parallel), then linked into one shared library
next to this file, where `_lib.py` loads it. The build always recompiles: it is cheap (seconds per file)
and it is the "does it build" check.
"""

from __future__ import annotations

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

try:
    from . import _lib
except ImportError:  # run as a script: this directory is on sys.path
    import _lib

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR.parent / "csrc"
INCLUDE = PKG_DIR.parent.parent / "include"
BUILD_DIR = PKG_DIR.parent / "_build"
LIB_PATH = PKG_DIR / "libbpt_amd.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Packed FP32 (v_pk_fma_f32 and friends) stays off: plain float code is compiled to scalar VALU ops.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the ROCm toolchain is needed to build libbpt_amd.so")
    return path


def _compile(src: Path, obj: Path, defines: tuple[str, ...] = ()) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, *(f"-D{d}" for d in defines), f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
    if src.name == "capi.hip":  # the sources' hash, which the loader compares with the tree's
        cmd.insert(1, f'-DBPT_SOURCE_HASH="{_lib.source_hash()}"')
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{proc.stderr}")
    noise = "is not a recognized feature for this target"
    for line in proc.stderr.splitlines():
        if line.strip() and noise not in line:
            print(line)


def build(verbose: bool = True, defines: tuple[str, ...] = (), out: Path | None = None) -> Path:
    """Compile every csrc/*.hip for gfx950 and link libbpt_amd.so. Returns the library path.

    `defines` (NAME=VALUE) override the kernels' compile-time tuning constants; `out` writes the library
    elsewhere (tuning builds), leaving the in-tree one alone.
    """
    lib_path = LIB_PATH if out is None else Path(out)
    build_dir = BUILD_DIR if out is None else lib_path.parent / (lib_path.stem + "_objs")
    build_dir.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objects = [build_dir / (s.stem + ".o") for s in sources]
    workers = min(len(sources), int(os.environ.get("MAX_JOBS", "8")), 16)
    with ThreadPoolExecutor(max_workers=max(workers, 1)) as pool:
        list(pool.map(lambda so: _compile(so[0], so[1], tuple(defines)), zip(sources, objects)))
    tmp = lib_path.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"linking libbpt_amd.so failed:\n{proc.stderr}")
    os.replace(tmp, lib_path)
    if verbose:
        print(f"built {lib_path} from {len(sources)} sources for {ARCH}" + (f" with {list(defines)}" if defines else ""))
    return lib_path


if __name__ == "__main__":
    build()
