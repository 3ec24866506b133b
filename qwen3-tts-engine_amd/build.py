"""Build recipe for the q3attn HIP library (gfx950): ``python build.py`` or ``build()``.

Compiles every ``csrc/*.hip`` with hipcc for gfx950 and links ``q3attn/libq3attn.so`` in-tree, so
the built library travels with the source tree.  Object files go to ``_build/`` (git-ignored).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "q3attn", "libq3attn.so")
# HBM probes (measurement infrastructure for bench.py --workload probe), a library of their own
PROBE_SRC = os.path.join(HERE, "probe", "hbm_probe.hip")
PROBE_OUT = os.path.join(HERE, "q3attn", "libq3probe.so")
BUILD = os.path.join(HERE, "_build")
ARCH = os.environ.get("Q3A_OFFLOAD_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-mcode-object-version=5",
    "-Wall", "-Wno-unused-function",
    # no packed-fp32 instructions in generated code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in VGPRs: loop-carried accumulators that VALU code also touches are otherwise
    # copied VGPR <-> AGPR around every MFMA block
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
]


def scratch_users(remarks: str) -> list[str]:
    """Kernels whose resource-usage remarks report scratch (private) memory per lane: a register array the
    compiler could not keep in VGPRs, which turns every access into a memory round trip."""
    users, name = [], None
    for ln in remarks.splitlines():
        m = re.search(r"remark: Function Name: (\S+)", ln)
        if m:
            name = m.group(1)
            continue
        m = re.search(r"remark:\s+ScratchSize \[bytes/lane\]: (\d+)", ln)
        if m and int(m.group(1)) > 0:
            users.append(f"{name} ({m.group(1)} B/lane)")
    return users


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(os.path.dirname(src)) + "_" + os.path.basename(src) + ".o")
    cmd = [HIPCC, *CFLAGS, "-Rpass-analysis=kernel-resource-usage", "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    lines = [ln for ln in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in ln]
    # drop the remarks and the source excerpts the compiler prints under them
    msg = "\n".join(ln for ln in lines if "remark:" not in ln and not re.match(r"^\s*(\d+\s+)?\|", ln))
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{msg}")
    spills = scratch_users("\n".join(lines))
    if spills:
        raise RuntimeError(f"{src}: kernels using scratch memory: {', '.join(spills)}")
    if msg.strip():
        print(msg, file=sys.stderr)
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs) + 1)) as ex:
        objs = list(ex.map(_compile, srcs + [PROBE_SRC]))
    for out, parts in ((OUT, objs[:-1]), (PROBE_OUT, objs[-1:])):
        tmp = out + ".tmp"
        cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *parts, "-o", tmp]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
        os.replace(tmp, out)
        if verbose:
            print(f"built {out}")
    return OUT


if __name__ == "__main__":
    build(verbose=True)
