"""Builds libvcpp_attn.so (the gfx950 paged-attention library) in-tree.

Usage: python vllm-cpp_amd/build.py   (or __graft_entry__.build()).
Every HIP source is compiled for gfx950 only, with packed-fp32 instruction
selection disabled, and linked into one shared library next to this file.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB = os.path.join(HERE, "libvcpp_attn.so")
SOURCES = ["csrc/decode.hip", "csrc/prefill.hip", "csrc/dense.hip", "csrc/kv_write.hip", "csrc/qk_prep.hip", "csrc/api.cpp",
           "csrc/profile.cpp", "csrc/noalloc.cpp", "host/kv_cache_manager.cpp", "host/paged_attention.cpp"]
HEADERS = ["host/host_util.h", "csrc/decode.h", "csrc/prefill.h", "csrc/prefill_body.h", "csrc/dense.h", "csrc/kv_write.h", "csrc/qk_prep.h", "csrc/device_common.h", "csrc/profile.h"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"),
    "-I", os.path.join(HERE, "csrc"),
]

# Per-source additions.  prefill.hip: LLVM's max-ILP machine scheduler orders
# the MFMA / exp / LDS-read mix of the prefill loop about 2 % faster on
# config 3 than the default occupancy-driven one (measured A/B on MI355X).
SOURCE_FLAGS = {
    "csrc/prefill.hip": ["-mllvm", "--amdgpu-sched-strategy=max-ilp"],
}


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError("build failed: %s\n%s" % (" ".join(cmd), err))
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(verbose=False, out=LIB, defines=()):
    """Compiles every source and links `out`; `defines` (e.g. "NAME=1") are
    passed as -D options, for building variants of the kernels side by side."""
    objs = []
    tag = "" if out == LIB else "_" + os.path.splitext(os.path.basename(out))[0]
    bdir = os.path.join(HERE, "_build" + tag)
    os.makedirs(bdir, exist_ok=True)
    dflags = ["-D" + d for d in defines]
    cmds = []
    for src in SOURCES:
        obj = os.path.join(bdir, os.path.basename(src) + ".o")
        lang = ["-x", "hip"]
        cmds.append([HIPCC] + FLAGS + SOURCE_FLAGS.get(src, []) + dflags + lang +
                    ["-c", os.path.join(HERE, src), "-o", obj])
        objs.append(obj)
    # One hipcc per source, run side by side (each is single-threaded).
    with ThreadPoolExecutor(max_workers=min(len(cmds), os.cpu_count() or 1, 8)) as ex:
        for f in [ex.submit(_run, c, verbose) for c in cmds]:
            f.result()
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", out] + objs, verbose)
    return out


GATHER_LIB = os.path.join(HERE, "libvcpp_attn_gather.so")


def build_gather_checker(verbose=False):
    """libvcpp_attn_gather.so: the same sources with -DVCPP_GATHER_DUMP, whose
    kernels also record the (block, slot) each (sequence, position) is loaded
    from (tests/test_gather_gpu.py).  A checker build; the product is LIB."""
    return build(verbose, out=GATHER_LIB, defines=["VCPP_GATHER_DUMP"])


def build_host_test(verbose=False):
    """tests/cpp/host_api_test: the C++ BlockPool / KVCacheManager /
    paged_attention checks, linked against this library and the CPU oracle
    (oracle/liboracle.so, which must be built first)."""
    src = os.path.join(ROOT, "tests", "cpp", "host_api_test.cpp")
    out = os.path.join(ROOT, "tests", "cpp", "host_api_test")
    _run([HIPCC, "--offload-arch=gfx950", "-O2", "-std=c++17", "-Wall",
          "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROOT, "oracle"), src,
          "-o", out, "-L", HERE, "-lvcpp_attn", "-L", os.path.join(ROOT, "oracle"), "-loracle",
          "-Wl,-rpath,$ORIGIN/../../vllm-cpp_amd", "-Wl,-rpath,$ORIGIN/../../oracle"], verbose)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
