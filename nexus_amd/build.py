"""Build the native library in-tree: nexus_amd/libnexus_hip_attn.so (gfx950).

Every HIP/C++ source under nexus_amd/csrc and nexus_amd/host is compiled with hipcc for
gfx950 only, with packed-FP32 instructions disabled, and linked into one shared library
that exports the C ABI of include/nexus_hip_attn.h plus the C++ host backend.

    python -m nexus_amd.build            # build (always recompiles)
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
BUILD_DIR = PKG / "_build"
LIB_NAME = "libnexus_hip_attn.so"
LIB_PATH = PKG / LIB_NAME
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    # packed FP32 (v_pk_*_f32) stays off in every kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # no NaN semantics are relied on (masking uses infinities): max/min need no input
    # canonicalisation
    "-fno-honor-nans",
    "-Wall",
    "-Wno-unused-function",
    f"-I{ROOT / 'include'}",
    f"-I{PKG / 'csrc'}",
    f"-I{PKG / 'host'}",
]


def sources() -> list[Path]:
    out = []
    for sub in ("csrc", "host"):
        d = PKG / sub
        if d.is_dir():
            out += sorted(p for p in d.iterdir() if p.suffix in (".hip", ".cpp"))
    return out


def _compile(src: Path) -> Path:
    obj = BUILD_DIR / (src.parent.name + "_" + src.stem + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
    if src.suffix == ".hip":
        cmd[1:1] = ["-x", "hip"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (res.stderr or "").splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{' '.join(cmd)}\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = False) -> Path:
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    BUILD_DIR.mkdir(exist_ok=True)
    srcs = sources()
    jobs = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(srcs)} sources")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
