"""Builds `liblinnet_quant_hip.so` from `linnet_amd/csrc` with hipcc for gfx950.

Each source is compiled to an object in parallel, then linked into the shared
library in-tree (`linnet_amd/_lib/`), written to a temporary name and renamed
so that a process already holding the library never sees a half-written file.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE / "csrc"
INCLUDE = PACKAGE.parent / "include"
LIBDIR = PACKAGE / "_lib"
LIBRARY = LIBDIR / "liblinnet_quant_hip.so"
ARCH = "gfx950"

# -packed-fp32-ops keeps hipcc from emitting packed f32 VALU instructions (the
# host pass warns it does not know the feature; that is harmless).
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-ffp-contract=off",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


# Per-source extra flags. The skinny and GEMV kernels feed every MFMA result
# straight to VALU math, so their accumulators belong in VGPRs (no accvgpr
# moves). A kernel without AGPRs also gets the whole register budget as VGPRs;
# one with AGPRs has it split in half, and the GEMV kernels then spill.
EXTRA = {name: ["-mllvm", "-amdgpu-mfma-vgpr-form"] for name in ("int4.hip", "int4_gemv.hip", "fp8_block.hip")}


def hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found: the HIP toolchain (ROCm) is required to build")
    return found


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))


def _compile(source: Path, objdir: Path) -> Path:
    obj = objdir / (source.stem + ".o")
    lang = ["-x", "hip"] if source.suffix in (".hip", ".cpp") else []
    cmd = [hipcc(), *FLAGS, *EXTRA.get(source.name, []), f"-I{INCLUDE}", *lang, "-c",
           str(source), "-o", str(obj)]
    done = subprocess.run(cmd, capture_output=True, text=True)
    if done.returncode != 0:
        raise RuntimeError(f"hipcc failed on {source.name}:\n{done.stdout}\n{done.stderr}")
    return obj


def _link(objects: list[Path], target: Path) -> None:
    staged = LIBDIR / f".{target.name}.{os.getpid()}.tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(staged), *map(str, objects)]
    done = subprocess.run(cmd, capture_output=True, text=True)
    if done.returncode != 0:
        raise RuntimeError(f"linking {target.name} failed:\n{done.stdout}\n{done.stderr}")
    os.replace(staged, target)


def build(verbose: bool = False) -> Path:
    """Compiles every source under csrc/ and links the library; returns its path."""
    LIBDIR.mkdir(parents=True, exist_ok=True)
    with tempfile.TemporaryDirectory(prefix="lnq_build_") as tmp:
        objdir = Path(tmp)
        srcs = sources()
        workers = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
        with ThreadPoolExecutor(max_workers=workers) as pool:
            objects = list(pool.map(lambda src: _compile(src, objdir), srcs))
        _link(objects, LIBRARY)
    if verbose:
        print(f"built {LIBRARY}", file=sys.stderr)
    return LIBRARY


if __name__ == "__main__":
    build(verbose=True)
