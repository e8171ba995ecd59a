"""Build libmira_hip.so for gfx950 in-tree (official-mira-llm_amd/mira_amd/lib/).

    python official-mira-llm_amd/build.py [-j N]

Every translation unit under csrc/ is compiled by hipcc for --offload-arch=gfx950 only, in
parallel, and linked into one shared library with a C-ABI (include/mira_hip.h). Packed FP32
instructions are switched off for all device code.
"""
from __future__ import annotations

import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "mira_amd", "lib")
LIBRARY = os.path.join(LIBDIR, "libmira_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wall", "-Wno-unused-function", "-Wno-unused-variable"]


def sources():
    return sorted(os.path.join(CSRC, name) for name in os.listdir(CSRC) if name.endswith(".hip"))


def source_hash():
    """sha256 over every csrc file and the public header: compiled into the library and checked
    by the loader, so a library built from other sources is refused rather than run."""
    import hashlib

    digest = hashlib.sha256()
    header = os.path.join(os.path.dirname(HERE), "include", "mira_hip.h")
    for path in sorted(os.path.join(CSRC, n) for n in os.listdir(CSRC)) + [header]:
        digest.update(os.path.basename(path).encode())
        with open(path, "rb") as handle:
            digest.update(handle.read())
    return digest.hexdigest()[:16]


def compile_one(source, objdir, digest):
    obj = os.path.join(objdir, os.path.basename(source) + ".o")
    command = [HIPCC, *FLAGS, f"-DMIRA_SOURCE_HASH=\"{digest}\"", "-c", source, "-o", obj]
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed on {source}:\n{result.stdout}\n{result.stderr}")
    return obj


def build(jobs=None, verbose=True):
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), os.cpu_count() or 1, 8)
    digest = source_hash()
    with concurrent.futures.ThreadPoolExecutor(jobs) as pool:
        objects = list(pool.map(lambda s: compile_one(s, objdir, digest), srcs))
    tmp = LIBRARY + ".tmp"
    command = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objects, "-lhipblaslt",
               "-o", tmp]
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"link failed:\n{result.stdout}\n{result.stderr}")
    os.replace(tmp, LIBRARY)
    shutil.rmtree(objdir, ignore_errors=True)
    if verbose:
        print(f"built {LIBRARY} from {len(srcs)} sources", flush=True)
    return LIBRARY


if __name__ == "__main__":
    parser = argparse.ArgumentParser()
    parser.add_argument("-j", type=int, default=None)
    args = parser.parse_args()
    try:
        build(args.j)
    except RuntimeError as error:
        print(error, file=sys.stderr)
        sys.exit(1)
