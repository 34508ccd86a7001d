"""Build ``libsimplicial_mi355x.so`` in-tree with hipcc for gfx950.

``python -m archlab_amd.build`` (with ``next-gen-arch_amd`` on ``sys.path``)
compiles every ``csrc/*.hip`` translation unit in parallel and links the
shared library next to this file.  The library exports only the C ABI of
``include/simplicial_mi355x.h``.
"""

from __future__ import annotations

import concurrent.futures
import glob
import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(HERE), "csrc")
OUT = os.path.join(HERE, "libsimplicial_mi355x.so")
ARCH = os.environ.get("SA_OFFLOAD_ARCH", "gfx950")

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 generation (those forms have
# produced silent wrong results on the target pool); the host pass warns that
# it does not know the feature, which is harmless.
# -fvisibility=hidden: only the C ABI (declared with default visibility in
# the header) is exported, so two builds loaded into one process (or another
# library) cannot interpose each other's internal functions.
# -mno-amdgpu-ieee / -fno-honor-nans: fmax without NaN canonicalisation; the
# kernels never produce NaN from finite inputs and use -inf explicitly.
COMMON = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-mcode-object-version=5",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-mno-amdgpu-ieee", "-fno-honor-nans", "-Wall", "-Wno-unused-function",
          "-fvisibility=hidden"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build the library)")


def _compile(src: str, obj: str) -> tuple[str, int, str]:
    cmd = [hipcc(), *COMMON, "-c", src, "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    log = "\n".join(line for line in (proc.stdout + proc.stderr).splitlines()
                    if "packed-fp32-ops" not in line)
    return src, proc.returncode, log


def build(verbose: bool = False) -> str:
    """Compile and link; returns the library path.  Raises on any failure."""
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    with tempfile.TemporaryDirectory(prefix="sa_build_") as tmp:
        objs = [os.path.join(tmp, os.path.basename(s) + ".o") for s in sources]
        with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(sources))) as pool:
            results = list(pool.map(_compile, sources, objs))
        failed = [(s, log) for s, rc, log in results if rc != 0]
        if verbose:
            for s, _, log in results:
                if log.strip():
                    print(f"[{os.path.basename(s)}]\n{log}", file=sys.stderr)
        if failed:
            msg = "\n".join(f"{os.path.basename(s)}:\n{log}" for s, log in failed)
            raise RuntimeError(f"hipcc failed:\n{msg}")
        tmp_out = OUT + ".tmp"
        cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp_out]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"link failed:\n{proc.stdout}{proc.stderr}")
        os.replace(tmp_out, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
