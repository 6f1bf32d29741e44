"""Build libvmonarch_gfx950.so in-tree with hipcc (gfx950 only).

    python -m vmonarch_amd.build          # compile every source, link the library

Objects go to vmonarch_amd/_build/, the library next to this file.  The library carries only
the gfx950 code object; it links the HIP runtime by soname (libamdhip64.so.7), so a process
that imported torch first keeps a single HIP runtime (torch's).
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libvmonarch_gfx950.so")
SOURCES = ["capi.hip", "fea_fwd.hip", "fea_bwd.hip", "lstep.hip", "lstep_mb.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-mcode-object-version=5",
    # no packed-fp32 instructions: ordinary float code only
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # no IEEE-mode NaN quieting: max/min need no canonicalising ops (inputs are finite)
    "-mno-amdgpu-ieee", "-fno-honor-nans",
    "-I", os.path.join(os.path.dirname(HERE), "include"),
]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError("command failed:\n" + " ".join(cmd) + "\n" + r.stdout)
    return r.stdout


def build(verbose=False, jobs=None):
    os.makedirs(BUILD, exist_ok=True)
    srcs = [s for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    objs = [os.path.join(BUILD, os.path.splitext(s)[0] + ".o") for s in srcs]
    cmds = [[HIPCC, *FLAGS, "-c", os.path.join(CSRC, s), "-o", o] for s, o in zip(srcs, objs)]
    with ThreadPoolExecutor(max_workers=jobs or min(8, len(cmds))) as ex:
        for out in ex.map(_run, cmds):
            if verbose and out.strip():
                print(out)
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp])
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
