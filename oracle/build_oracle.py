"""Build recipe for the oracle's C restatement (test infrastructure only).

Compiles ``oracle/encode_ref.c`` with gcc into ``oracle/_build/libss_oracle.so``.
Strict IEEE float64 (``-ffp-contract=off``, no fast-math) so the C oracle's
rounding is deterministic.  The reference itself (Python + MLX) has no C
sources, so there is no ``oracle/_ref`` build.
"""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(OUT_DIR, "libss_oracle.so")


def build(verbose: bool = False) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    cmd = ["gcc", "-O2", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off",
           "-std=c11", os.path.join(HERE, "encode_ref.c"), "-o", LIB + ".tmp"]
    if verbose:
        print(" ".join(cmd))
    subprocess.run(cmd, check=True)
    os.replace(LIB + ".tmp", LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
