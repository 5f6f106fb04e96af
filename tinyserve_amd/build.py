"""Compile ``csrc/*.hip`` for gfx950 into ``libtinyserve_amd.so`` next to this file.

The library is built in-tree with ``hipcc`` (no JIT cache), so the built file travels
with the repository snapshot to the GPU machine. Usage::

    python -m tinyserve_amd.build          # or tinyserve_amd.build.build()
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD_DIR = PKG / "_build"
LIB_NAME = "libtinyserve_amd.so"
ARCH = "gfx950"

# -packed-fp32-ops off: no v_pk_{add,mul,fma}_f32 are generated from float code.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]  # fmt: skip


# Per-source extra flags. prefill.hip: no NaN handling is needed in its softmax (masked
# scores are -inf, never NaN), and without it fmaxf skips the NaN-quieting v_max that IEEE
# mode otherwise puts before every max of an MFMA result.
EXTRA_FLAGS = {"prefill.hip": ["-fno-honor-nans"]}


def hipcc() -> str:
    """Path of hipcc: $HIPCC, then PATH, then /opt/rocm/bin."""
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: set HIPCC or install ROCm")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path, verbose: bool) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, *EXTRA_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature: harmless.
    noise = "is not a recognized feature for this target"
    err = "\n".join(ln for ln in proc.stderr.splitlines() if noise not in ln)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every source (always; no staleness check) and link the shared library."""
    BUILD_DIR.mkdir(exist_ok=True)
    srcs = sources()
    with ThreadPoolExecutor(max_workers=min(len(srcs), os.cpu_count() or 1)) as pool:
        objs = list(pool.map(lambda s: _compile(s, verbose), srcs))
    out = PKG / LIB_NAME
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    tmp.replace(out)  # atomic: a process that already mapped the old file keeps it
    return out


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
