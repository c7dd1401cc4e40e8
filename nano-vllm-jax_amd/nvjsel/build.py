"""Build libnvjsel.so in-tree with hipcc for gfx950.

``python nano-vllm-jax_amd/nvjsel/build.py`` (or ``build()``) compiles every
``csrc/*.hip`` translation unit in parallel and links the shared library next
to this file, where ``nvjsel._lib`` loads it.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR.parent / "csrc"
INCLUDE = PKG_DIR.parent.parent / "include"
LIB_PATH = PKG_DIR / "libnvjsel.so"
OBJ_DIR = PKG_DIR.parent / "_build"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("NVJSEL_ARCH", "gfx950")

# -packed-fp32-ops off: hand-off of packed fp32 ALU forms is avoided on this
# pool; correctly rounded fp32 division/sqrt and IEEE denormals are required
# for bit-exact temperature scaling.
COMMON_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-fast-math",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}",
]


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path) -> Path:
    obj = OBJ_DIR / (src.stem + ".o")
    # NVJSEL_STRICT_ORDERING=1: order the last-block reductions with the HIP
    # memory model's acquire-release ticket instead of data dependencies
    # (csrc/nvjsel_device.h, ticket_add)
    extra = ["-DNVJSEL_STRICT_ORDERING=1"] if os.environ.get("NVJSEL_STRICT_ORDERING") == "1" else []
    cmd = [HIPCC, *COMMON_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stderr[-6000:]}")
    return obj


def build(verbose: bool = False) -> Path:
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-6000:]}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
