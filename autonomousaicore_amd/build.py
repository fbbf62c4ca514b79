"""Builds the native library autonomousaicore_amd/libaic_hip.so for gfx950 with hipcc.

Every .hip / .cpp under csrc/ is compiled in parallel into _build/ and linked into one
shared library.  `python -m autonomousaicore_amd.build` (or __graft_entry__.build())
always recompiles; loading the package never compiles.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libaic_hip.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

# -packed-fp32-ops: keep the compiler from emitting packed fp32 VALU ops (v_pk_*_f32).
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON = ["-O3", "-std=c++20", "-fPIC", f"--offload-arch={ARCH}", "-Wall", "-Wno-unused-parameter",
          "-Wno-unused-function", "-I", os.path.join(ROOT, "include")]


def sources() -> list[str]:
    out = []
    for ext in ("hip", "cpp"):
        out += glob.glob(os.path.join(CSRC, "**", f"*.{ext}"), recursive=True)
    return sorted(out)


def _obj(src: str) -> str:
    rel = os.path.relpath(src, CSRC).replace(os.sep, "_")
    return os.path.join(BUILD, rel + ".o")


# Per-file code generation options.  attention.hip: MFMAs in the VGPR form, so that the
# backward's long-lived dK/dV accumulators are not copied between VGPRs and AGPRs around every
# MFMA of the inner loop (the AGPR form's register assignment does that for these kernels).
FILE_FLAGS = {"attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}


def _compile(src: str) -> tuple[str, int, str]:
    obj = _obj(src)
    cmd = [HIPCC, *COMMON, *DEVICE_FLAGS, *FILE_FLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj]
    p = subprocess.run(cmd, capture_output=True, text=True)
    msg = "\n".join(l for l in (p.stdout + p.stderr).splitlines() if "packed-fp32-ops" not in l)
    return src, p.returncode, msg


def build(jobs: int | None = None, verbose: bool = False) -> str:
    if not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(16, max(1, (os.cpu_count() or 4)))
    failed = []
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for src, rc, msg in ex.map(_compile, srcs):
            if rc != 0:
                failed.append((src, msg))
            elif verbose and msg.strip():
                print(msg, file=sys.stderr)
    if failed:
        for src, msg in failed:
            print(f"--- {src}\n{msg}", file=sys.stderr)
        raise RuntimeError(f"{len(failed)} source(s) failed to compile")
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *[_obj(s) for s in srcs]]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError("link failed:\n" + p.stdout + p.stderr)
    shutil.move(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
