"""Build libtreemoe_amd.so (gfx950) and the C restatement of the oracle.

Run as ``python -m treemoe_spec_amd._build``.  Every source is compiled on each
call; objects are compiled in parallel and linked in-tree, so the shared
library travels with the source tree to the GPU host.
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
CSRC = PKG / "csrc"
LIB = PKG / "libtreemoe_amd.so"
OBJ_DIR = PKG / "_build"
ORACLE_C = ROOT / "oracle" / "c"
ORACLE_LIB = ROOT / "oracle" / "liboracle_c.so"

HIP_SOURCES = ["capi.hip", "op1_route.hip", "op1_gemm.hip", "op1_prefill.hip", "op4_verify.hip",
               "tree_attn.hip"]
ARCH = os.environ.get("TREEMOE_AMD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: install ROCm or set HIPCC")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def build_library() -> Path:
    hipcc = _hipcc()
    OBJ_DIR.mkdir(exist_ok=True)
    objs = [OBJ_DIR / (Path(s).stem + ".o") for s in HIP_SOURCES]
    cmds = [[hipcc, *HIPCC_FLAGS, "-c", str(CSRC / s), "-o", str(o)]
            for s, o in zip(HIP_SOURCES, objs)]
    with ThreadPoolExecutor(max_workers=min(len(cmds), 4)) as pool:
        list(pool.map(_run, cmds))
    tmp = LIB.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
          *map(str, objs)])
    os.replace(tmp, LIB)
    return LIB


def build_oracle() -> Path:
    """CPU restatement: strict IEEE single precision, no contraction."""
    cc = os.environ.get("CC", "gcc")
    tmp = ORACLE_LIB.with_suffix(".so.tmp")
    _run([cc, "-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off",
          "-fno-fast-math", "-Wall", "-o", str(tmp), str(ORACLE_C / "tm_oracle.c"),
          "-lm"])
    os.replace(tmp, ORACLE_LIB)
    return ORACLE_LIB


def build_fast_binding() -> Path:
    """_tmfast: CPython-API calls of the per-step op4 entry points, linked
    against libtreemoe_amd.so in the same directory."""
    import sysconfig

    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    out = PKG / ("_tmfast" + suffix)
    tmp = out.with_suffix(".tmp")
    cxx = os.environ.get("CXX", "g++")
    _run([cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall",
          f"-I{sysconfig.get_paths()['include']}", "-o", str(tmp), str(CSRC / "pyfast.cpp"),
          f"-L{PKG}", "-ltreemoe_amd", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, out)
    return out


def build_all() -> None:
    build_oracle()
    build_library()
    build_fast_binding()


if __name__ == "__main__":
    build_all()
    print(f"built {LIB} and {ORACLE_LIB}")
