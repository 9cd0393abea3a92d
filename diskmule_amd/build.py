"""Build the gfx950 library ``libdmhip.so`` from ``csrc/`` with hipcc, and
the measurement-only ``libdmhip_diag.so`` (launch-floor probes,
``include/dmhip_diag.h``) from ``csrc/diag/``.

Every HIP source is compiled for gfx950 only, with FMA contraction off (all
fused multiply-adds in the kernels are explicit) and without packed-FP32
instruction selection.  The build fails if any kernel uses scratch (private
memory): register spills cost bandwidth, and the first launch of such a
kernel makes the runtime allocate scratch backing, which the
allocation-free entry point promises never happens.
"""
from __future__ import annotations

import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libdmhip.so")
DIAG_LIB = os.path.join(HERE, "libdmhip_diag.so")
SOURCES = ["runtime.hip", "dispatch.hip", "kernels_simple.hip", "kernels_qmv.hip", "kernels_qmv8.hip",
           "kernels_gemm.hip", "expert_cache.hip", "kernels_dense.hip", "attention.hip",
           "kernels_safetensor.hip"]
DIAG_SOURCES = ["diag/probes.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
         "-Rpass-analysis=kernel-resource-usage"]
# Extra hipcc flags per source file (none at present).
SOURCE_FLAGS: dict = {}


def build(verbose: bool = False, jobs: int = 6) -> str:
    objdir = os.path.join(HERE, "_build")
    os.makedirs(os.path.join(objdir, "diag"), exist_ok=True)
    procs = []
    objs = {LIB: [], DIAG_LIB: []}
    for lib, sources in ((LIB, SOURCES), (DIAG_LIB, DIAG_SOURCES)):
        for src in sources:
            path = os.path.join(CSRC, src)
            obj = os.path.join(objdir, src + ".o")
            objs[lib].append(obj)
            cmd = [HIPCC, *FLAGS, *SOURCE_FLAGS.get(src, []), "-c", path, "-o", obj]
            procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
            if len(procs) >= jobs:
                _drain(procs, verbose)
    _drain(procs, verbose)
    for lib, lib_objs in objs.items():
        tmp = lib + ".tmp"
        subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *lib_objs], check=True)
        os.replace(tmp, lib)
    return LIB


def scratch_users(text: str) -> list:
    """Kernels whose resource-usage remarks report scratch bytes per lane."""
    users, name = [], None
    for line in text.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name = m.group(1)
        m = re.search(r"ScratchSize \[bytes/lane\]: (\d+)", line)
        if m and int(m.group(1)) > 0:
            users.append(f"{name} ({m.group(1)} bytes/lane)")
    return users


def _drain(procs, verbose):
    failed = None
    for cmd, p in procs:
        out, _ = p.communicate()
        text = out.decode(errors="replace")
        # hipcc's host pass does not know the packed-fp32 feature: harmless;
        # the resource-usage remarks are read, not shown.
        lines = [l for l in text.splitlines()
                 if "packed-fp32-ops" not in l and "remark:" not in l and not re.match(r"^\s*(\d+\s*)?\|", l)]
        if verbose or p.returncode:
            sys.stderr.write("\n".join(lines) + ("\n" if lines else ""))
        if p.returncode and failed is None:
            failed = cmd
        spills = scratch_users(text)
        if spills and failed is None:
            sys.stderr.write("kernels using scratch:\n  " + "\n  ".join(spills) + "\n")
            failed = cmd
    procs.clear()
    if failed:
        raise RuntimeError("hipcc failed: " + " ".join(failed))


if __name__ == "__main__":
    print(build(verbose=True))
