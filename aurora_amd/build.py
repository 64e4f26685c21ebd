"""Builds libaurora_hip.so (HIP kernels + C ABI) in-tree for gfx950 with hipcc.

Each source under ``aurora_amd/csrc`` is compiled to an object in
``aurora_amd/_build`` (in parallel), then linked into ``aurora_amd/libaurora_hip.so``.
Cross-compiles without a GPU.
"""
from __future__ import annotations

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT_DIR = PKG / "_build"
LIB = PKG / "libaurora_hip.so"
INCLUDE = PKG.parent / "include"
# Roofline ceiling probes (a measurement aid for bench.py, not the C ABI).
PROBE_SRC = PKG / "probes" / "ceilings.hip"
PROBE_LIB = PKG / "libaurora_ceilings.so"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# Packed-FP32 instructions are disabled for all device code (the compiler
# would otherwise emit v_pk_* forms from ordinary float code).
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def sources() -> list[Path]:
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


def _compile(src: Path) -> Path:
    obj = OUT_DIR / (src.stem + ".o")
    cmd = [HIPCC, *DEVICE_FLAGS, f"-I{INCLUDE}", "-c", str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd.insert(1, "-x")
        cmd.insert(2, "hip")
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")
    return obj


def build(verbose: bool = False, jobs: int = 8) -> Path:
    """Compile every source and link the shared library. Always rebuilds."""
    if not Path(HIPCC).exists() and shutil.which("hipcc") is None:
        raise RuntimeError("hipcc not found: cannot build libaurora_hip.so")
    OUT_DIR.mkdir(exist_ok=True)
    srcs = sources()
    with ThreadPoolExecutor(max_workers=min(jobs, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    build_probes()
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources, and {PROBE_LIB.name}")
    return LIB


def build_probes() -> Path:
    """Compile the ceiling probes into their own shared library."""
    tmp = PROBE_LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, *DEVICE_FLAGS, "-shared", str(PROBE_SRC), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {PROBE_SRC.name}:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, PROBE_LIB)
    return PROBE_LIB


if __name__ == "__main__":
    build(verbose=True)
