"""Builds the in-tree shared libraries of the MI355X attention path.

    lib/libsixi_attn.so   gfx950 HIP kernels + the C ABIs of include/sixi_attn.h,
                          include/sixi_kv.h, include/sixi_plan.h,
                          include/sixi_layer.h and include/sixi_gdn.h (hipcc)
    lib/libsixi_synth.so  seeded synthetic workload generator used by bench.py and tests (g++)

Run as ``python sixi-asi_amd/build.py`` or through ``__graft_entry__.build()``.  Every call
recompiles; objects go to ``_build/`` (not committed), libraries to ``lib/``.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import pathlib
import shutil
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
ROOT = PKG.parent
INCLUDE = ROOT / "include"
CSRC = PKG / "csrc"
HOST = PKG / "host"
LIB = PKG / "lib"
OBJ = PKG / "_build"

ARCH = os.environ.get("SIXI_OFFLOAD_ARCH", "gfx950")
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # gfx950: keep hand-written and compiler-generated code off the packed-FP32 VALU ops
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]
# Per-source flags.  fa_decode.hip: MFMA accumulators in VGPR form (the software-pipelined
# step loop keeps O in the 256 VGPRs and its operands in AGPRs; in AGPR form the compiler
# copies the 96 accumulator registers across every iteration).  gdn_verify.hip: the same, for
# the chunked kernel's state, which is an MFMA operand and accumulator at once (in AGPR form it
# took 52 AGPRs and 244 VGPRs).
FILE_FLAGS = {"fa_decode.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=true"],
              "gdn_verify.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=true"]}


def flags_for(src: str) -> list[str]:
    return [*HIP_FLAGS, *FILE_FLAGS.get(src, [])]


HIP_SOURCES = ["fa_decode.hip", "fa_prefill.hip", "fa_mask.hip", "fa_q8_stage.hip", "kv_write.hip", "sixi_attn_abi.cpp", "sixi_kv_abi.cpp",
               "sixi_kv_pool.cpp",
               "sixi_plan.cpp", "layer_prologue.hip", "sixi_layer_abi.cpp",
               "gdn_verify.hip", "sixi_gdn_abi.cpp"]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and pathlib.Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the gfx950 kernels cannot be built")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{out}")


def build_attn(jobs: int | None = None) -> pathlib.Path:
    hipcc = _hipcc()
    OBJ.mkdir(exist_ok=True)
    LIB.mkdir(exist_ok=True)
    objs = []
    cmds = []
    for src in HIP_SOURCES:
        obj = OBJ / (src.replace(".", "_") + ".o")
        objs.append(obj)
        lang = ["-x", "hip"] if src.endswith(".cpp") else []
        cmds.append([hipcc, *flags_for(src), *lang, "-c", str(CSRC / src), "-o", str(obj)])
    with cf.ThreadPoolExecutor(max_workers=jobs or min(8, len(cmds))) as ex:
        list(ex.map(_run, cmds))
    out = LIB / "libsixi_attn.so"
    tmp = LIB / "libsixi_attn.so.tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, out)
    return out


def build_synth() -> pathlib.Path:
    LIB.mkdir(exist_ok=True)
    out = LIB / "libsixi_synth.so"
    tmp = LIB / "libsixi_synth.so.tmp"
    _run(["g++", "-O2", "-fPIC", "-shared", "-std=c++17", "-fopenmp", "-ffp-contract=off", "-mf16c",
          f"-I{HOST}", "-o", str(tmp), str(HOST / "synth.cpp")])
    os.replace(tmp, out)
    return out


def build(jobs: int | None = None) -> list[pathlib.Path]:
    return [build_attn(jobs), build_synth()]


if __name__ == "__main__":
    for p in build():
        print(p)
    sys.exit(0)
