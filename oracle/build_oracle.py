"""Compile the C oracle (test infrastructure) into oracle/liboracle.so with gcc.

The reference implementation is pure Python, so there is no reference C/C++
source to compile into oracle/_ref; only this restatement is built.
-ffp-contract=off keeps every multiply and add separately rounded, as the
eager elementwise ops the oracle restates round them.
"""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
SOURCE = HERE / "kvr_oracle.c"
OUTPUT = HERE / "liboracle.so"


def build(verbose: bool = False) -> Path:
    cmd = ["gcc", "-O2", "-std=c99", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math", "-Wall",
           str(SOURCE), "-o", str(OUTPUT), "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    result = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if result.returncode != 0:
        raise RuntimeError("oracle build failed:\n" + result.stdout)
    return OUTPUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
