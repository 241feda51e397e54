"""Builds ``libasrattn.so`` (the HIP kernels and their C ABI) for gfx950.

The library is compiled in place, next to this file, with ``hipcc`` and no
PyTorch dependency; it is loaded with ctypes (:mod:`asrback_amd._lib`).

    python -m asrback_amd.build
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
SOURCES = sorted((PACKAGE / "csrc").glob("*.hip"))
HEADERS = sorted((PACKAGE / "csrc").glob("*.hpp")) + [ROOT / "include" / "asrattn.h"]
LIBRARY = PACKAGE / "libasrattn.so"
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-shared",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Packed fp32 VALU instructions stay off: the compiler would otherwise
    # form v_pk_* from ordinary float code.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm under /opt/rocm)")


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    result = subprocess.run(cmd, capture_output=True, text=True)
    output = "\n".join(
        line
        for line in (result.stdout + result.stderr).splitlines()
        if "packed-fp32-ops" not in line  # the host pass does not know the feature
    )
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed ({result.returncode}):\n{output}")
    if verbose and output.strip():
        print(output, flush=True)


def build(verbose: bool = False) -> Path:
    """Compile every kernel source (one hipcc per source, in parallel) and
    link them into ``libasrattn.so``; return its path."""
    if not SOURCES:
        raise RuntimeError(f"no HIP sources under {PACKAGE / 'csrc'}")
    includes = [f"-I{ROOT / 'include'}", f"-I{PACKAGE / 'csrc'}"]
    compile_flags = [flag for flag in FLAGS if flag != "-shared"]
    tmp = LIBRARY.with_suffix(f".so.tmp{os.getpid()}")
    with tempfile.TemporaryDirectory(prefix="asrattn_build_") as work:
        objects = [str(Path(work) / (source.stem + ".o")) for source in SOURCES]
        jobs = [[hipcc(), *compile_flags, *includes, "-c", str(source), "-o", obj]
                for source, obj in zip(SOURCES, objects)]
        workers = max(1, min(len(jobs), int(os.environ.get("MAX_JOBS", "0")) or os.cpu_count() or 1))
        with concurrent.futures.ThreadPoolExecutor(workers) as pool:
            for future in [pool.submit(_run, job, verbose) for job in jobs]:
                future.result()
        try:
            _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objects, "-o", str(tmp)], verbose)
        except BaseException:
            tmp.unlink(missing_ok=True)
            raise
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    path = build(verbose="-q" not in sys.argv)
    print(path)
