"""Build libmhc_amd.so (gfx950) in-tree with hipcc.

Usage: ``python flagos-mhc_amd/build.py`` or ``build()`` from Python.  Every
``csrc/*.hip`` file is compiled to an object in parallel, then linked into
``FlagOS_mhc/libmhc_amd.so`` next to the Python package that loads it.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "FlagOS_mhc", "libmhc_amd.so")
ARCH = "gfx950"

# -packed-fp32-ops off: hipcc must not form v_pk_*_f32 from scalar code.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libmhc_amd.so)")


def _run(cmd):
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # the host pass warns that it does not know the packed-fp32 feature: harmless
    lines = [l for l in p.stdout.splitlines() if "packed-fp32-ops" not in l]
    return p.returncode, "\n".join(lines)


def build(verbose: bool = False) -> str:
    hipcc = _hipcc()
    sources = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))
    tmp = tempfile.mkdtemp(prefix="mhc_build_")
    try:
        objs, jobs = [], []
        with cf.ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
            for src in sources:
                obj = os.path.join(tmp, src[:-4] + ".o")
                objs.append(obj)
                cmd = [hipcc, *HIPCC_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
                jobs.append((src, ex.submit(_run, cmd)))
            for src, fut in jobs:
                rc, out = fut.result()
                if out.strip() and (verbose or rc):
                    print(out, file=sys.stderr)
                if rc:
                    raise RuntimeError(f"hipcc failed on {src}")
        tmp_so = OUT + ".tmp"
        # --no-undefined: a kernel whose host stub the compiler did not emit
        # fails here rather than when the library is loaded
        rc, out = _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,--no-undefined", *objs, "-o", tmp_so])
        if rc:
            print(out, file=sys.stderr)
            raise RuntimeError("link of libmhc_amd.so failed")
        os.replace(tmp_so, OUT)
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
