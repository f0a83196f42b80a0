"""Build libpaged_attention_amd.so for gfx950 with hipcc (no CMake, no JIT).

Each .hip source is compiled to an object under csrc/_build/ in parallel and
the objects are linked into ``<package>/libpaged_attention_amd.so``, which is
what ``_native.load_library`` opens.  ``python csrc/build.py`` or
``build()`` from the package both run it; every call recompiles.
"""

from __future__ import annotations

import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

CSRC = Path(__file__).resolve().parent
PACKAGE_DIR = CSRC.parent
REPO_ROOT = PACKAGE_DIR.parent
INCLUDE_DIR = REPO_ROOT / "include"
BUILD_DIR = CSRC / "_build"
LIBRARY_NAME = "libpaged_attention_amd.so"
LIBRARY_PATH = PACKAGE_DIR / LIBRARY_NAME
OFFLOAD_ARCH = "gfx950"

SOURCES = ["abi.hip", "plan.cpp", "pack.hip", "cache_write.hip", "decode.hip", "generic.hip", "prefill.hip",
           "prefill256.hip", "prefill_f32.hip", "copy_blocks.hip", "calibrate.hip"]

HIP_FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={OFFLOAD_ARCH}",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Packed-fp32 VALU forms are kept out of every device object.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


# Per-source additions: the MFMA prefill for heads of 64-128 keeps its
# accumulators in architectural VGPRs (no AGPR copies around the softmax
# rescale); the one for heads of 256 (one wave per SIMD) leaves them to the
# AGPRs.
EXTRA_FLAGS = {"prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH") or os.environ.get("ROCM_HOME") or "/opt/rocm"
    path = Path(rocm) / "bin" / "hipcc"
    if path.exists():
        return str(path)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found: a ROCm toolchain is required to build the HIP path")
    return found


def _compile(hipcc: str, source: str) -> Path:
    obj = BUILD_DIR / (Path(source).stem + ".o")
    cmd = [hipcc, *HIP_FLAGS, *EXTRA_FLAGS.get(source, []), f"-I{INCLUDE_DIR}", f"-I{CSRC}", "-c",
           str(CSRC / source), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {source}:\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every source for gfx950 and link the shared library."""
    hipcc = _hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4)) as pool:
        objects = list(pool.map(lambda s: _compile(hipcc, s), SOURCES))
    tmp = LIBRARY_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIBRARY_PATH)
    if verbose:
        print(f"built {LIBRARY_PATH}")
    return LIBRARY_PATH


def build_revision(rev: str, out: Path) -> Path:
    """Build the library from the sources of git revision ``rev`` into
    ``out`` (a measurement aid: ``bench.py --ab-library out`` times it in
    alternation with the in-tree build).  The revision's own build script
    compiles its own tree, extracted with ``git archive`` into a temporary
    directory."""
    out = Path(out).resolve()
    with tempfile.TemporaryDirectory() as tmp:
        archive = subprocess.run(["git", "-C", str(REPO_ROOT), "archive", rev], capture_output=True, check=True)
        subprocess.run(["tar", "-x", "-C", tmp], input=archive.stdout, check=True)
        script = Path(tmp) / PACKAGE_DIR.name / "csrc" / "build.py"
        proc = subprocess.run([sys.executable, str(script)], capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"building {rev} failed:\n{proc.stdout}\n{proc.stderr}")
        shutil.copy2(Path(tmp) / PACKAGE_DIR.name / LIBRARY_NAME, out)
    return out


if __name__ == "__main__":
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--rev", help="build this git revision's sources instead of the tree's")
    ap.add_argument("--out", help="with --rev: where to put the library")
    args = ap.parse_args()
    if args.rev:
        if not args.out:
            ap.error("--rev needs --out")
        print(f"built {build_revision(args.rev, Path(args.out))}")
    else:
        build(verbose=True)
    sys.exit(0)
