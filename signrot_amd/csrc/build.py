"""Build libsignrot_hip.so (all HIP kernels + the C ABI) for gfx950.

Usage: python -m signrot_amd.csrc.build   (or signrot_amd.csrc.build.build())

Every .hip file in this directory is compiled with hipcc for gfx950 only,
in parallel, and linked into signrot_amd/_lib/libsignrot_hip.so.  The
library is built in-tree so it travels with the source tree; it is
git-ignored.
"""
import concurrent.futures as cf
import os
import pathlib
import shutil
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent
PKG = HERE.parent
ROOT = PKG.parent
OUT_DIR = PKG / "_lib"
LIB = OUT_DIR / "libsignrot_hip.so"
OBJ_DIR = ROOT / "_build" / "obj"

ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    # no FMA contraction: the quantizers and the dequant epilogue must keep
    # the reference's separate roundings; wanted FMAs are written explicitly
    "-ffp-contract=off",
    # packed fp32 (v_pk_*_f32) instructions stay off on this pool
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _compile(src, obj):
    cmd = [hipcc(), *FLAGS, "-I", str(ROOT / "include"), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the gfx feature flag; drop that noise
    err = "\n".join(l for l in res.stderr.splitlines()
                    if "packed-fp32-ops" not in l or "error" in l.lower())
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    return err


def build(verbose=True):
    sources = sorted(HERE.glob("*.hip"))
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    OUT_DIR.mkdir(parents=True, exist_ok=True)
    objs = [OBJ_DIR / (s.stem + ".o") for s in sources]
    with cf.ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        futs = {ex.submit(_compile, s, o): s for s, o in zip(sources, objs)}
        for f in cf.as_completed(futs):
            msg = f.result()
            if verbose and msg.strip():
                print(f"[{futs[f].name}]\n{msg}", file=sys.stderr)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB.relative_to(ROOT)} from {len(sources)} sources")
    return LIB


if __name__ == "__main__":
    build()
