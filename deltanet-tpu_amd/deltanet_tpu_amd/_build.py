"""Build the gfx950 HIP library in-tree with hipcc (no torch extension, no JIT cache)."""

from __future__ import annotations

import os
import shutil
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.dirname(HERE)                      # deltanet-tpu_amd/
REPO_ROOT = os.path.dirname(PKG_ROOT)
CSRC = os.path.join(PKG_ROOT, "csrc")
INCLUDE = os.path.join(REPO_ROOT, "include")
SOURCES = ("dn_prefill.hip", "dn_decode.hip", "dn_backward.hip")
OUT = os.path.join(HERE, "libdeltanet_amd.so")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build deltanet_tpu_amd)")


def build(arch: str = "gfx950", out: str = OUT, extra=(), jobs: int = 3) -> str:
    """Compile every HIP source for `arch` and link the shared library `out`."""
    objs = []
    procs = []
    for src in SOURCES:
        obj = os.path.join(HERE, src.replace(".hip", f".{arch}.o"))
        cmd = [hipcc(), f"--offload-arch={arch}", "-O3", "-std=c++17", "-fPIC", "-c",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               "-I", INCLUDE, "-I", CSRC, *extra, os.path.join(CSRC, src), "-o", obj]
        procs.append((subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT), src))
        objs.append(obj)
        if len(procs) >= jobs:
            _wait(procs.pop(0))
    for p in procs:
        _wait(p)
    tmp = out + ".tmp"
    cmd = [hipcc(), f"--offload-arch={arch}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout.decode(errors="replace"))
    os.replace(tmp, out)
    for o in objs:
        os.remove(o)
    return out


def _wait(pair):
    p, src = pair
    outp, _ = p.communicate()
    if p.returncode != 0:
        text = outp.decode(errors="replace")
        raise RuntimeError(f"hipcc failed for {src}:\n{text}")


if __name__ == "__main__":
    print(build())
