"""Build the gfx950 HIP library libd3w8a8.so in-tree (d3trt_amd/libd3w8a8.so).

Each csrc/*.hip file is compiled for gfx950 only, in parallel, then linked as a
shared library exporting the C ABI of include/d3w8a8.h. Flags that matter for
results:
  -ffp-contract=off      no a*b+c fusion (the eager torch chain rounds twice)
  (default) correctly rounded fp32 division / sqrt
  -Xclang -target-feature -Xclang -packed-fp32-ops   no packed-fp32 VALU ops
  -Werror=inline-asm     inline asm the compiler cannot honour (a reserved register in a
                         clobber list) fails the build
"""

from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
PKG = os.path.join(HERE, "d3trt_amd")
BUILD = os.path.join(HERE, "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
    "-Werror=inline-asm",  # e.g. a reserved register (m0) in a clobber list, which the compiler ignores
]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src).replace(".hip", ".o"))
    cmd = [HIPCC, *FLAGS, "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    # the GEMM instantiation files take the longest: start them first
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")),
                     key=lambda s: (not os.path.basename(s).startswith("gemm_"), s))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        objs = list(ex.map(_compile, sources))
    out = os.path.join(PKG, "libd3w8a8.so")
    tmp = out + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(out)
    return out


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
