"""Build recipe for libvcx.so (gfx950 only).

Each .hip translation unit is compiled by hipcc to a position-independent
object in parallel, then linked into lib/libvcx.so next to this file. Flags:
  --offload-arch=gfx950           CDNA4 code objects only
  -ffp-contract=off               no implicit a*b+c fusion: every rounding in the
                                  byte contract is explicit (fmaf where intended)
  -target-feature -packed-fp32-ops  no v_pk_{add,mul,fma}_f32 (the host pass warns
                                  that it does not know the feature; harmless)
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
LIB = HERE / "lib" / "libvcx.so"
SOURCES = ["vcx_abi.hip", "vcx_prep.hip", "vcx_group.hip", "vcx_attn.hip"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; the HIP extension cannot be built")


COMMON = ["-O3", "-std=c++17", "--offload-arch=gfx950", "-fPIC", "-ffp-contract=off",
          "-fno-gpu-rdc", "-Wall", "-Wno-unused-function",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def build(verbose: bool = False) -> Path:
    obj_dir = HERE / "_build"
    obj_dir.mkdir(exist_ok=True)
    cc = hipcc()

    def compile_one(src: str) -> Path:
        obj = obj_dir / (Path(src).stem + ".o")
        cmd = [cc, *COMMON, "-c", str(CSRC / src), "-o", str(obj)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src}:\n{res.stdout}\n{res.stderr}")
        if verbose:
            noise = "not a recognized feature"
            msg = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
            if msg.strip():
                print(msg)
        return obj

    with cf.ThreadPoolExecutor(max_workers=min(4, len(SOURCES))) as pool:
        objs = list(pool.map(compile_one, SOURCES))
    LIB.parent.mkdir(exist_ok=True)
    tmp = LIB.with_suffix(".so.tmp%d" % os.getpid())
    cmd = [cc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
