"""Builds libmlxr.so (gfx950) in-tree from mlx-runner_amd/csrc with hipcc.

Usage: python mlx-runner_amd/build.py [-j N]
The library lands at mlx-runner_amd/libmlxr.so; objects under mlx-runner_amd/_build/.
"""
import argparse
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libmlxr.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("MLXR_ARCH", "gfx950")

FLAGS = [
    "-x", "hip", f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable", "-Wno-unused-value", "-Wno-unused-result",
    "-I", os.path.join(ROOT, "include"), "-I", SRC,
]


def sources():
    return sorted(f for f in os.listdir(SRC) if f.endswith((".hip", ".cpp")))


def compile_one(name):
    src = os.path.join(SRC, name)
    obj = os.path.join(OUT, name + ".o")
    cmd = [HIPCC, *FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {name}:\n{out}")
    return obj, out


def build(jobs=8, verbose=False):
    os.makedirs(OUT, exist_ok=True)
    objs = []
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for obj, out in ex.map(compile_one, sources()):
            objs.append(obj)
            if verbose and out.strip():
                print(out)
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp, "-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=8)
    ap.add_argument("-v", action="store_true")
    a = ap.parse_args()
    print(build(a.j, a.v))
    sys.exit(0)
