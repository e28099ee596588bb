"""Build libmanta_rocm.so (HIP, gfx950) and libmanta_synth.so in-tree.

Usage: python -m manta_amd.build  (or manta_amd.build.build()).
Every call recompiles; objects go to manta_amd/_build/.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libmanta_rocm.so")
SYNTH = os.path.join(HERE, "libmanta_synth.so")

HIP_SOURCES = ["kernels_score.hip", "kernels_ref.hip", "kernels_topk.hip", "kernels_mq.hip", "kernels_mq4.hip", "kernels_mq8.hip",
               "kernels_embed.hip", "kernels_encoder.hip", "kernels_exec.hip", "kernels_dense.hip", "noalloc.hip", "runtime.cpp", "mll.cpp",
               "module.cpp", "program.cpp"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # packed f32 VALU forms stay off: some of their forms have given wrong
    # results on this hardware without any error
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-I" + os.path.join(ROOT, "include"),
    "-I" + CSRC,
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: libmanta_rocm.so cannot be built")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError("build failed: %s\n%s" % (" ".join(cmd), out))
    if out.strip():
        sys.stderr.write(out + "\n")


def build_rocm() -> str:
    hipcc = _hipcc()
    os.makedirs(OBJ, exist_ok=True)
    objs = []
    cmds = []
    for src in HIP_SOURCES:
        obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
        lang = ["-x", "hip"] if src.endswith(".hip") else []
        cmds.append([hipcc] + HIPCC_FLAGS + lang + ["-c", os.path.join(CSRC, src), "-o", obj])
        objs.append(obj)
    with cf.ThreadPoolExecutor(max_workers=min(4, len(cmds))) as ex:
        list(ex.map(_run, cmds))
    tmp = LIB + ".tmp"
    _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs + ["-lpthread"])
    os.replace(tmp, LIB)
    return LIB


def build_synth() -> str:
    gxx = shutil.which("g++") or "g++"
    tmp = SYNTH + ".tmp"
    _run([gxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-fopenmp", "-I" + CSRC,
          os.path.join(CSRC, "synth.cpp"), "-o", tmp])
    os.replace(tmp, SYNTH)
    return SYNTH


def build() -> None:
    build_synth()
    build_rocm()


if __name__ == "__main__":
    build()
    print(LIB)
    print(SYNTH)
