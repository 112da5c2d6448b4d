"""Build recipe for libmas_kernels.so, the C-ABI library of the gfx950 layer kernels, and for
libmas_bench.so, the benchmark's memory skeletons.

Every ``csrc/*.hip`` file is compiled for gfx950 with hipcc (in parallel), then linked into one
shared library next to this file; ``bench_csrc/*.hip`` likewise into the benchmark's library. The
output is written under a temporary name and renamed, so a process that already mapped the
previous library is not disturbed.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
CSRC_DIR = PACKAGE_DIR / "csrc"
BENCH_CSRC_DIR = PACKAGE_DIR / "bench_csrc"
INCLUDE_DIR = PACKAGE_DIR.parent / "include"
LIBRARY_NAME = "libmas_kernels.so"
LIBRARY_PATH = PACKAGE_DIR / LIBRARY_NAME
BENCH_LIBRARY_PATH = PACKAGE_DIR / "libmas_bench.so"
ARCH = "gfx950"

# -ffp-contract=off keeps every fp32 product and sum separately rounded, so the kernels' arithmetic
# follows the written operation order. The packed-fp32 feature is switched off for the device
# pass (hipcc's host pass warns that it does not know the feature name).
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-result",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the ROCm toolchain is required to build the kernels")
    return path


def sources(directory: Path = CSRC_DIR) -> list[Path]:
    return sorted(directory.glob("*.hip"))


def _compile(src: Path, obj: Path) -> tuple[Path, str]:
    cmd = [hipcc(), *DEVICE_FLAGS, f"-I{INCLUDE_DIR}", "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    return obj, proc.stderr


def build_library(verbose: bool = False, jobs: int | None = None, directory: Path = CSRC_DIR,
                  library: Path = LIBRARY_PATH) -> Path:
    """Compiles and links the HIP sources of ``directory`` into ``library``; returns its path."""
    srcs = sources(directory)
    if not srcs:
        raise RuntimeError(f"no HIP sources under {directory}")
    jobs = jobs or min(len(srcs), max(1, int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))), 8)
    with tempfile.TemporaryDirectory(prefix="mas_build_") as tmp:
        objs = [Path(tmp) / (s.stem + ".o") for s in srcs]
        with ThreadPoolExecutor(max_workers=jobs) as pool:
            results = list(pool.map(_compile, srcs, objs))
        if verbose:
            for obj, err in results:
                lines = [ln for ln in err.splitlines() if "packed-fp32-ops" not in ln]
                if lines:
                    print(f"[{obj.stem}]", "\n".join(lines))
        staged = library.parent / f".{library.name}.tmp{os.getpid()}"
        cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(staged)]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
        os.replace(staged, library)
    if verbose:
        print(f"built {library} from {len(srcs)} sources")
    return library


def build_bench_library(verbose: bool = False) -> Path:
    """The benchmark's memory skeletons (not part of the kernel library)."""
    return build_library(verbose, directory=BENCH_CSRC_DIR, library=BENCH_LIBRARY_PATH)


if __name__ == "__main__":
    build_library(verbose=True)
    build_bench_library(verbose=True)
