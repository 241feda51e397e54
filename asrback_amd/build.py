"""Builds ``libasrattn.so`` (the HIP kernels and their C ABI) for gfx950.

The library is compiled in place, next to this file, with ``hipcc`` and no
PyTorch dependency; it is loaded with ctypes (:mod:`asrback_amd._lib`).

    python -m asrback_amd.build
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
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


def build(verbose: bool = False) -> Path:
    """Compile every kernel source into ``libasrattn.so`` and return its path."""
    if not SOURCES:
        raise RuntimeError(f"no HIP sources under {PACKAGE / 'csrc'}")
    tmp = LIBRARY.with_suffix(f".so.tmp{os.getpid()}")
    cmd = [
        hipcc(),
        *FLAGS,
        f"-I{ROOT / 'include'}",
        f"-I{PACKAGE / 'csrc'}",
        *map(str, SOURCES),
        "-o",
        str(tmp),
    ]
    if verbose:
        print(" ".join(cmd), flush=True)
    result = subprocess.run(cmd, capture_output=True, text=True)
    output = "\n".join(
        line
        for line in (result.stdout + result.stderr).splitlines()
        if "packed-fp32-ops" not in line  # the host pass does not know the feature
    )
    if result.returncode != 0:
        tmp.unlink(missing_ok=True)
        raise RuntimeError(f"hipcc failed ({result.returncode}):\n{output}")
    if verbose and output.strip():
        print(output, flush=True)
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    path = build(verbose="-q" not in sys.argv)
    print(path)
