"""Build recipe for ``libsrdit_hip.so``: one hipcc invocation, gfx950 only.

``python -m sr_dit.build`` (with ``dreamx-creator_amd`` on ``sys.path``) or
``build()`` compiles every ``csrc/*.hip`` into the shared library next to the
``sr_dit`` package.  hipcc cross-compiles for gfx950 without a GPU present.
"""
from __future__ import annotations

import glob
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)            # dreamx-creator_amd/
REPO = os.path.dirname(ROOT)
CSRC = os.path.join(ROOT, "csrc")
INCLUDE = os.path.join(REPO, "include")
OUT = os.path.join(PKG_DIR, "libsrdit_hip.so")

ARCH = "gfx950"
# Packed fp32 VALU ops are switched off for all device code.
HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-Wno-unused-command-line-argument"]
# Per-source additions.  The window kernels keep their MFMA results and
# accumulators in the VGPR form: a lazily rescaled O accumulator is otherwise
# mirrored between AGPRs and VGPRs every step.  The GEMM keeps the default.
FILE_FLAGS = {"window_attn.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
              "window_group.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
              "dense_attn.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
              # the fused elementwise kernels round after every operation, as
              # torch's separate kernels do: no multiply-add contraction
              "fused.hip": ["-ffp-contract=off"]}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libsrdit_hip.so)")


def sources():
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")))


def _run(cmds, verbose):
    """Run compiler commands in parallel; raise with the filtered stderr on failure."""
    noise = "is not a recognized feature for this target"
    procs = []
    for cmd in cmds:
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE,
                                            text=True)))
    errors = []
    for cmd, p in procs:
        _, err = p.communicate()
        err = "\n".join(l for l in err.splitlines() if noise not in l)
        if p.returncode != 0:
            errors.append(f"{os.path.basename(cmd[-3])}: hipcc failed ({p.returncode}):\n{err}")
        elif verbose and err.strip():
            print(err, file=sys.stderr)
    if errors:
        raise RuntimeError("\n".join(errors))


def build(verbose: bool = False) -> str:
    """Compile the library; returns its path.  Always recompiles."""
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objdir = os.path.join(PKG_DIR, "_obj")
    os.makedirs(objdir, exist_ok=True)
    cc = hipcc()
    objs, cmds = [], []
    for src in srcs:
        obj = os.path.join(objdir, os.path.basename(src) + ".o")
        objs.append(obj)
        cmds.append([cc, *HIP_FLAGS, *FILE_FLAGS.get(os.path.basename(src), []),
                     f"-I{INCLUDE}", f"-I{CSRC}", "-c", src, "-o", obj])
    _run(cmds, verbose)
    tmp = OUT + ".tmp"
    _run([[cc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]], verbose)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
