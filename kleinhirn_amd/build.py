"""Builds libkh_hip.so (the gfx950 kernels and the C ABI of include/kh_hip.h) in-tree with hipcc."""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libkh_hip.so")
SOURCES = ["runner.hip", "gemm.hip", "attention.hip", "rowops.hip"]
HOST_SOURCES = ["manifest.cpp", "postprocess.cpp", "sched.cpp"]  # host code only: the system C++ compiler
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "-shared", "--offload-arch=gfx950",
    # packed FP32 instructions stay off (some of their forms gave wrong results on these boxes)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


def build(verbose: bool = False) -> str:
    """Compiles every source into one shared library (always recompiles)."""
    objs = []
    procs = []
    for src in SOURCES:
        obj = os.path.join(CSRC, "_build", src.replace(".hip", ".o"))
        os.makedirs(os.path.dirname(obj), exist_ok=True)
        cmd = [HIPCC, *[f for f in FLAGS if f != "-shared"], "-c", os.path.join(CSRC, src), "-o", obj]
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
        objs.append(obj)
    for src in HOST_SOURCES:
        obj = os.path.join(CSRC, "_build", src.replace(".cpp", ".o"))
        os.makedirs(os.path.dirname(obj), exist_ok=True)
        cmd = ["g++", "-O3", "-std=c++17", "-fPIC", "-Wall", "-c", os.path.join(CSRC, src), "-o", obj]
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
        objs.append(obj)
    failed = False
    for cmd, p in procs:
        out, _ = p.communicate()
        lines = [l for l in out.splitlines() if "packed-fp32-ops" not in l]
        if p.returncode != 0 or (verbose and lines):
            sys.stderr.write(" ".join(cmd) + "\n" + "\n".join(lines) + "\n")
        failed |= p.returncode != 0
    if failed:
        raise RuntimeError("hipcc failed")
    tmp = LIB + ".tmp"
    subprocess.run([HIPCC, "-shared", "-fPIC", "--offload-arch=gfx950", *objs, "-o", tmp], check=True)
    os.replace(tmp, LIB)
    build_addon()
    write_build_info()
    return LIB


def write_build_info() -> None:
    """kleinhirn_amd/build_info.json: the commit the library was built from (and whether the tree
    held uncommitted changes), read by bench.py where the tree has no git history."""
    import json
    info = {"commit": None, "dirty": None}
    try:
        info["commit"] = subprocess.run(["git", "-C", ROOT, "rev-parse", "--short=12", "HEAD"], capture_output=True,
                                        text=True, check=True).stdout.strip()
        st = subprocess.run(["git", "-C", ROOT, "status", "--porcelain", "--untracked-files=no"],
                            capture_output=True, text=True, check=True).stdout
        info["dirty"] = bool(st.strip())
    except (OSError, subprocess.CalledProcessError):
        pass
    with open(os.path.join(HERE, "build_info.json"), "w") as fh:
        json.dump(info, fh)


ADDON = os.path.join(HERE, "node", "kh_addon.node")
NODE_INCLUDE = "/usr/include/node"


def build_addon() -> str | None:
    """kh_addon.node (plain N-API C) against libkh_hip.so, when the Node headers are present."""
    if not os.path.exists(os.path.join(NODE_INCLUDE, "node_api.h")):
        return None
    subprocess.run(["gcc", "-O2", "-shared", "-fPIC", "-std=c11", "-Wall", f"-I{NODE_INCLUDE}",
                    "-DNODE_GYP_MODULE_NAME=kh_addon", os.path.join(HERE, "node", "kh_addon.c"),
                    "-o", ADDON, f"-L{HERE}", "-lkh_hip", "-Wl,-rpath,$ORIGIN/.."], check=True)
    return ADDON


if __name__ == "__main__":
    print(build(verbose=True))
