"""Builds the gfx950 HIP backend, libllrs_hip.so, in-tree.

Every HIP source is compiled for gfx950 only, with packed-FP32 instruction
selection switched off (-Xclang -target-feature -Xclang -packed-fp32-ops);
host-only C++ (the quantizers) is compiled with -ffp-contract=off so its f32
arithmetic keeps the reference's evaluation order.

    python llama.rs_amd/build.py [--jobs N] [--stamps]

--stamps also builds libllrs_hip_stamps.so: the same library with the
persistent decode kernel recompiled with -DLLRS_STAMPS, which records
wall-clock stamps per phase and workgroup (read by phase_profile.py).  The
product library is unchanged.
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
PER_FILE = {"quantize.hip": ["-ffp-contract=off"], "quantize_host.cpp": ["-ffp-contract=off"],
            "synth.cpp": ["-ffp-contract=off"], "model.cpp": ["-ffp-contract=off"]}


def sources():
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


STAMPS_LIB = PKG / "libllrs_hip_stamps.so"
STAMPED = "decode_persistent.hip"


def compile_one(src: pathlib.Path, stamps: bool = False) -> pathlib.Path:
    obj = BUILD / (src.name + (".stamps.o" if stamps else ".o"))
    cmd = [HIPCC] + COMMON
    if src.suffix == ".hip":
        cmd += HIP_FLAGS + ["-x", "hip"]
    cmd += PER_FILE.get(src.name, [])
    if stamps:
        cmd += ["-DLLRS_STAMPS"]
    cmd += ["-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (res.stdout + res.stderr).splitlines()
                    if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {src.name}\n{' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)
    return obj


def link(objs, out: pathlib.Path) -> None:
    tmp = out.with_suffix(".so.tmp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp)] + \
          [str(o) for o in objs] + ["-lpthread"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed\n{' '.join(cmd)}\n{res.stdout}{res.stderr}")
    os.replace(tmp, out)


def build(jobs: int | None = None, stamps: bool = False) -> pathlib.Path:
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 16)
    with cf.ThreadPoolExecutor(jobs) as ex:
        futs = [ex.submit(compile_one, s) for s in srcs]
        stamped = ex.submit(compile_one, CSRC / STAMPED, True) if stamps else None
        objs = [f.result() for f in futs]
        if stamped:
            stamped = stamped.result()
    link(objs, LIB)
    if stamped:
        link([stamped if o.name == STAMPED + ".o" else o for o in objs], STAMPS_LIB)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--stamps", action="store_true")
    args = ap.parse_args()
    print(build(args.jobs, args.stamps))
