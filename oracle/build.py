"""Build the oracle's C brute-force GEMM into oracle/libd3oracle.so (TEST ORACLE).

The reference is pure Python (no C/C++ source on this path), so there is no
reference library to compile into oracle/_ref; only this restatement is built.
"""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))


def build() -> str:
    src = os.path.join(HERE, "igemm.c")
    out = os.path.join(HERE, "libd3oracle.so")
    tmp = out + ".tmp"
    cmd = ["gcc", "-O3", "-fopenmp", "-fPIC", "-shared", "-o", tmp, src]
    subprocess.run(cmd, check=True)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build())
    sys.exit(0)
