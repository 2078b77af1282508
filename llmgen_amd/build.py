"""Build the gfx950 attention library in-tree: llmgen_amd/libllmgen_attn.so.

Every ``csrc/*.hip`` and ``csrc/*.cpp`` file is compiled with hipcc for gfx950 only and linked into one shared
library whose C-ABI is declared in ``include/*.h``.  Packed FP32 instructions are disabled for all device code
(``-target-feature -packed-fp32-ops``).  Run ``python -m llmgen_amd.build`` or call :func:`build`.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_NAME = "libllmgen_attn.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

INCLUDE = os.path.join(os.path.dirname(PKG_DIR), "include")
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    f"-I{INCLUDE}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _compile(src: str, obj: str) -> None:
    cmd = [HIPCC, *COMMON_FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature; that line is noise.
    noise = ("packed-fp32-ops", "is not a recognized feature")
    err = "\n".join(l for l in r.stderr.splitlines() if not any(n in l for n in noise))
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = True) -> str:
    """Compile every csrc/*.hip (device code) and csrc/*.cpp (host executor slice) and link libllmgen_attn.so.
    Returns the library path."""
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))
    obj_dir = os.path.join(PKG_DIR, "_build")
    os.makedirs(obj_dir, exist_ok=True)
    objs = [os.path.join(obj_dir, os.path.splitext(os.path.basename(s))[0] + ".o") for s in srcs]
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        list(ex.map(lambda so: _compile(*so), zip(srcs, objs)))
    tmp = LIB_PATH + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"[llmgen_amd.build] built {LIB_PATH} from {len(srcs)} sources for {ARCH}")
    return LIB_PATH


if __name__ == "__main__":
    build()
