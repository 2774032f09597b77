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
HEADERS = ["host/host_util.h", "csrc/decode.h", "csrc/prefill.h", "csrc/prefill_body.h", "csrc/prefill_wide.h",
           "csrc/prefill_wide_regs.h", "csrc/dense.h", "csrc/kv_write.h", "csrc/qk_prep.h", "csrc/device_common.h", "csrc/profile.h"]

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
# prefill.hip also keeps the compiler from spilling VGPRs into AGPRs: the wide
# prefill kernel holds its accumulators in AGPRs that only its inline assembly
# names (prefill_wide_regs.h), so no compiler value may be placed there.
SOURCE_FLAGS = {
    "csrc/prefill.hip": ["-mllvm", "--amdgpu-sched-strategy=max-ilp", "-mllvm", "-amdgpu-spill-vgpr-to-agpr=0"],
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


def check_agpr_use(src, extra, verbose=False):
    """The wide prefill kernels keep their accumulators in AGPRs that only
    their inline assembly names (csrc/prefill_wide_regs.h): fail the build if
    the compiler placed any value of its own in an AGPR of those kernels."""
    import re
    import tempfile
    with tempfile.TemporaryDirectory() as td:
        asm = os.path.join(td, "k.s")
        _run([HIPCC] + FLAGS + extra + ["-x", "hip", "--cuda-device-only", "-S", src, "-o", asm], verbose)
        text = open(asm).read()
    bad = []
    for m in re.finditer(r"^(_Z\w*prefill_wide_kernel\w*):\n(.*?)\ts_endpgm", text, re.S | re.M):
        in_asm = False
        for line in m.group(2).splitlines():
            if ";;#ASMSTART" in line:
                in_asm = True
            elif ";;#ASMEND" in line:
                in_asm = False
            elif not in_asm and re.match(r"\s+[a-z_0-9]+\s.*[\s,\[]a(\d|\[)", line):
                bad.append("%s: %s" % (m.group(1), line.strip()))
    if bad:
        raise RuntimeError("compiler-allocated AGPRs in the wide prefill kernels:\n" + "\n".join(bad[:20]))


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
    # One hipcc per source, run side by side (each is single-threaded), and
    # the AGPR check of the prefill kernels beside them.
    with ThreadPoolExecutor(max_workers=min(len(cmds) + 1, os.cpu_count() or 1, 8)) as ex:
        futs = [ex.submit(_run, c, verbose) for c in cmds]
        futs.append(ex.submit(check_agpr_use, os.path.join(HERE, "csrc/prefill.hip"),
                              SOURCE_FLAGS["csrc/prefill.hip"] + dflags, verbose))
        for f in futs:
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
