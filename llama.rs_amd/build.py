"""Builds the gfx950 HIP backend, libllrs_hip.so, in-tree.

Every HIP source is compiled for gfx950 only, with packed-FP32 instruction
selection switched off (-Xclang -target-feature -Xclang -packed-fp32-ops);
host-only C++ (the quantizers) is compiled with -ffp-contract=off so its f32
arithmetic keeps the reference's evaluation order.

    python llama.rs_amd/build.py [--jobs N]
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import pathlib
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libllrs_hip.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON = ["-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function", "-I", str(CSRC),
          "-I", str(PKG.parent / "include")]
HIP_FLAGS = ["--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-munsafe-fp-atomics"]
# The shared host/device encoders must evaluate f32 exactly as written.
PER_FILE = {"quantize.hip": ["-ffp-contract=off"], "synth.cpp": ["-ffp-contract=off"],
            "model.cpp": ["-ffp-contract=off"]}


def sources():
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


def compile_one(src: pathlib.Path) -> pathlib.Path:
    obj = BUILD / (src.name + ".o")
    cmd = [HIPCC] + COMMON
    if src.suffix == ".hip":
        cmd += HIP_FLAGS + ["-x", "hip"]
    cmd += PER_FILE.get(src.name, [])
    cmd += ["-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (res.stdout + res.stderr).splitlines()
                    if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {src.name}\n{' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)
    return obj


def build(jobs: int | None = None) -> pathlib.Path:
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 16)
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(compile_one, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp)] + \
          [str(o) for o in objs] + ["-lpthread"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed\n{' '.join(cmd)}\n{res.stdout}{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    args = ap.parse_args()
    print(build(args.jobs))
