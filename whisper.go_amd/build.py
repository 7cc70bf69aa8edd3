"""Build libwhisper_hip.so for gfx950 in-tree (whisper.go_amd/lib/).

Every source is compiled by hipcc for gfx950 only, with packed-fp32 code
generation disabled; objects go to whisper.go_amd/_build/ and are linked into
one shared library. Usage: python whisper.go_amd/build.py [-j N]
"""
import argparse
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIBDIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIBDIR, "libwhisper_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# the slowest first: the five instantiations of the batched persistent forward
SOURCES = ["wh_batch_q4_0.hip", "wh_batch_q4_1.hip", "wh_batch_q5_0.hip", "wh_batch_q5_1.hip", "wh_batch_q8_0.hip",
           "wh_mega.hip", "wh_kernels.hip", "wh_batch.hip", "wh_noalloc.hip", "wh_encoder.hip", "wh_seq.cpp",
           "wh_quant.cpp", "wh_model.cpp", "wh_encoder.cpp", "wh_api.cpp"]
CFLAGS = [
    "--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17", "-x", "hip",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result", "-Wno-unused-function",
]


def _compile(src):
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [HIPCC] + CFLAGS + ["-c", os.path.join(SRC, src), "-o", obj]
    p = subprocess.run(cmd, capture_output=True, text=True)
    msgs = [l for l in (p.stdout + p.stderr).splitlines() if "packed-fp32-ops" not in l]
    return src, obj, p.returncode, "\n".join(msgs)


def build(jobs=None, verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 4)
    objs = []
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for src, obj, rc, msg in ex.map(_compile, SOURCES):
            if msg.strip() and (verbose or rc):
                print(msg, file=sys.stderr)
            if rc:
                raise RuntimeError(f"hipcc failed on {src}")
            objs.append(obj)
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "--hip-link", "-o", tmp] + objs + ["-lpthread"]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode:
        print(p.stdout + p.stderr, file=sys.stderr)
        raise RuntimeError("link of libwhisper_hip.so failed")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=None)
    ap.add_argument("-v", action="store_true")
    a = ap.parse_args()
    print(build(a.j, a.v))
