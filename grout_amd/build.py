"""Builds grout_amd/libgrout_attn.so for gfx950 with hipcc (in-tree, so the
shared object travels with the source tree to the GPU machine).

    python -m grout_amd.build [--verbose] [--resource-usage]
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libgrout_attn.so")
ARCH = os.environ.get("GROUT_OFFLOAD_ARCH", "gfx950")

COMMON = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function",
    # packed fp32 VALU forms are kept out of generated code on this target
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
# (source, extra flags).  The norm/RoPE kernel must not contract mul+add:
# its K rows are checked bit for bit against a CPU restatement.
SOURCES = [
    ("qk_norm_rope.hip", ["-ffp-contract=off"]),
    ("attn_decode.hip", []),
    ("attn_prefill.hip", []),
    ("model_kernels.hip", []),
    ("quant_gemv.hip", []),
    ("api.cpp", ["-x", "hip"]),
    ("engine.cpp", ["-x", "hip"]),
    ("loader.cpp", ["-x", "hip"]),
    ("gguf.cpp", ["-x", "hip"]),
]
# Prefill projections are plain GEMMs: rocBLAS.
LIBS = ["-L/opt/rocm/lib", "-lrocblas", "-Wl,-rpath,/opt/rocm/lib"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the gfx950 HIP library cannot be built")


def _compile(src: str, extra: list[str], resource_usage: bool, verbose: bool) -> str:
    out = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *COMMON, *extra, "-c", os.path.join(CSRC, src), "-o", out]
    if resource_usage:
        cmd.append("-Rpass-analysis=kernel-resource-usage")
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    msgs = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                     if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{msgs}")
    if msgs.strip() and (verbose or resource_usage):
        print(msgs, flush=True)
    return out


def build(verbose: bool = False, resource_usage: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(lambda s: _compile(s[0], s[1], resource_usage, verbose), SOURCES))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, *LIBS, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB)
    _build_examples(verbose)
    return LIB


EXAMPLES = os.path.join(HERE, "examples")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")


def _build_examples(verbose: bool) -> None:
    """Host programs over the C++ API (include/grout.hpp), linked against the
    library just built; they find it next to them at run time."""
    cxx = shutil.which("g++") or shutil.which("c++")
    if cxx is None:
        raise RuntimeError("g++ not found: the C++ examples cannot be built")
    src = os.path.join(EXAMPLES, "generate.cpp")
    out = os.path.join(EXAMPLES, "grout_generate")
    cmd = [cxx, "-std=c++17", "-O2", "-Wall", "-Wextra", "-Werror", "-pedantic", f"-I{INCLUDE}",
           src, f"-L{HERE}", "-lgrout_attn", "-Wl,-rpath,$ORIGIN/..",
           "-Wl,-rpath-link,/opt/rocm/lib", "-o", out + ".tmp"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"example build failed:\n{r.stdout}{r.stderr}")
    os.replace(out + ".tmp", out)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("--resource-usage", action="store_true")
    a = ap.parse_args(argv)
    print(build(a.verbose, a.resource_usage))
    return 0


if __name__ == "__main__":
    sys.exit(main())
