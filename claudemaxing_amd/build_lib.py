"""Build the gfx950 kernel library `libclaudemaxing_amd.so` in-tree with hipcc.

Every `csrc/*.hip` file is compiled to an object for gfx950 only, then all objects are linked
into one shared library next to this file. Run as `python -m claudemaxing_amd.build_lib`.
"""

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
INCLUDE = PKG.parent / "include"
LIB_NAME = "libclaudemaxing_amd.so"
LIB_PATH = PKG / LIB_NAME
OBJ_DIR = PKG / "_build"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
    # packed fp32 instructions (v_pk_*_f32) stay off: only scalar fp32 VALU ops are emitted
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    # a struct of device pointers initialised with too few values leaves the rest null
    "-Werror=missing-field-initializers",
]


def _compile(src: Path) -> Path:
    obj = OBJ_DIR / (src.stem + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every HIP source and link the library. Always rebuilds."""
    if not Path(HIPCC).exists() and shutil.which("hipcc") is None:
        raise RuntimeError("hipcc not found: the gfx950 kernel library cannot be built")
    OBJ_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = max(1, min(len(sources), 8))
    with ThreadPoolExecutor(workers) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(sources)} sources", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
