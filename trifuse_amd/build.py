"""Build libtrifuse_moe.so (HIP, gfx950) in-tree with hipcc.

    python -m trifuse_amd.build          # compile every source, link the library

The library is written to trifuse_amd/lib/libtrifuse_moe.so. Each .hip file is
compiled to an object in trifuse_amd/lib/obj/ (in parallel), then linked.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIBDIR = PKG / "lib"
OBJDIR = LIBDIR / "obj"
LIBNAME = "libtrifuse_moe.so"
SOURCES = ["capi.hip", "route.hip", "group.hip", "gemv.hip", "decode.hip", "ggemm.hip", "combine.hip",
           "norm.hip", "dstream.hip", "dstream_f16.hip", "dstream_i8.hip",
           "dstream_f16_i8.hip"]
ARCH = "gfx950"

# -packed-fp32-ops off: hipcc must not form v_pk_{add,mul,fma}_f32 from float code.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{PKG.parent / 'include'}",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the HIP library cannot be built")
    return path


def _compile(src: str) -> Path:
    obj = OBJDIR / (Path(src).stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stdout}\n{res.stderr}")
    # The host pass does not know the packed-fp32 feature and says so; drop that line.
    noise = "-packed-fp32-ops' is not a recognized feature"
    msgs = [ln for ln in (res.stderr or "").splitlines() if noise not in ln]
    if msgs:
        sys.stderr.write("\n".join(msgs) + "\n")
    return obj


def build(verbose: bool = True) -> Path:
    OBJDIR.mkdir(parents=True, exist_ok=True)
    jobs = min(len(SOURCES), max(1, int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    out = LIBDIR / LIBNAME
    tmp = LIBDIR / (LIBNAME + ".tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    build()
