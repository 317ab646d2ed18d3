"""Build recipe for the gfx950 paged-attention library.

Compiles every HIP source under csrc/ with hipcc for gfx950 and links them into
engine/kernels/libpa_gfx950.so, next to the ctypes loader that opens it, and the
benchmark's read-bandwidth probes (probes/bw_probe.hip) into
probes/libbw_probe_gfx950.so. Object files go to _build/ at the repository root. Run directly
(``python vllm-inference-engine_amd/build.py``) or through
``__graft_entry__.build()``.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_ROOT = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO_ROOT / "include"
BUILD_DIR = REPO_ROOT / "_build"
LIB_PATH = PKG_DIR / "engine" / "kernels" / "libpa_gfx950.so"
PROBE_SRC = PKG_DIR / "probes" / "bw_probe.hip"
PROBE_LIB = PKG_DIR / "probes" / "libbw_probe_gfx950.so"

ARCH = "gfx950"

# Every HIP translation unit is compiled with these flags. Packed FP32 ops are
# switched off (-packed-fp32-ops); the host pass warns that it does not know
# the feature, which is harmless.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    "-Wall",
    "-Wno-unused-function",
]


# Extra flags per source file. The prefill attention kernel rescales its MFMA
# accumulators with vector ops; in the accumulator-register form every rescale
# copies them out and back, so its MFMAs use the VGPR form. Its score maxima
# would otherwise quiet possible signalling NaNs with an extra v_max per value
# (-fno-honor-nans; infinities, which the masking uses, keep their meaning).
FILE_FLAGS = {
    "pa_prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1", "-fno-honor-nans"],
}


def _hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build the library")
    return exe


def _sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile_one(src: Path) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [_hipcc(), *HIPCC_FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{proc.stdout}\n{proc.stderr}")
    return obj


def _link(objs: list[Path], lib: Path) -> None:
    tmp = lib.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs),
           "-Wl,-rpath,/opt/rocm/lib", "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link of {lib.name} failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, lib)


def build(verbose: bool = False) -> Path:
    """Compile all sources and link the shared libraries; returns the attention library's path."""
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    srcs = _sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs) + 1)) as ex:
        objs = list(ex.map(_compile_one, srcs + [PROBE_SRC]))
    _link(objs[:-1], LIB_PATH)
    _link(objs[-1:], PROBE_LIB)
    if verbose:
        print(f"built {LIB_PATH} from {len(srcs)} sources and {PROBE_LIB}", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
