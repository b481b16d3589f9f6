"""Build libmimir_prefixlm.so (the C-ABI HIP library) in-tree for gfx950.

Every HIP source under ``mimir_amd/csrc`` is compiled with hipcc for
``--offload-arch=gfx950`` and linked into ``mimir_amd/_lib/libmimir_prefixlm.so``.
No torch extension machinery is involved: the library exports only the
``extern "C"`` entry points declared in ``include/mimir_prefixlm.h`` and is loaded
with ctypes.  Run ``python -m mimir_amd.build`` (or ``__graft_entry__.build()``).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_DIR = PKG_DIR / "_lib"
LIB_PATH = LIB_DIR / "libmimir_prefixlm.so"
ARCH = "gfx950"

# Packed FP32 (v_pk_*_f32) is disabled: hipcc otherwise forms them from float2
# arithmetic.  The host pass warns that it does not know the feature; harmless.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fno-gpu-rdc",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]

# Per-source code generation options (none at present).
SOURCE_FLAGS: dict = {}

SOURCES = [
    "prefixlm_capi.hip",
    "prefixlm_fwd_bf16.hip",
    "prefixlm_bwd_bf16.hip",
    "prefixlm_bwd_dq_bf16.hip",
    "prefixlm_bwd_dq_ds_bf16.hip",
    "prefixlm_bwd_dkdv_bf16.hip",
    "prefixlm_bwd_dkdv_pair_bf16.hip",
    "prefixlm_f32.hip",
    "prefixlm_prologue.hip",
    "prefixlm_layer.hip",
    "prefixlm_cache_bf16.hip",
    "prefixlm_noalloc.hip",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found; set ROCM_PATH")
    return found


def _compile(src: Path, obj: Path) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, *SOURCE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = True) -> Path:
    """Compile every HIP source and link the shared library; returns its path."""
    obj_dir = LIB_DIR / "obj"
    obj_dir.mkdir(parents=True, exist_ok=True)
    objs = [obj_dir / (s.rsplit(".", 1)[0] + ".o") for s in SOURCES]
    with ThreadPoolExecutor(max_workers=min(4, len(SOURCES))) as ex:
        list(ex.map(lambda so: _compile(CSRC / so[0], so[1]), zip(SOURCES, objs)))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build()
