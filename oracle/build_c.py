"""Build recipe for the C oracle (test infrastructure): ``oracle/c/oracle.c`` ->
``oracle/_build/liboracle_c.so`` with gcc, IEEE-754 default arithmetic (no fast-math, no FMA
contraction)."""

from __future__ import annotations

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "c" / "oracle.c"
OUT = HERE / "_build" / "liboracle_c.so"


def build() -> Path:
    OUT.parent.mkdir(exist_ok=True)
    cmd = ["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math",
           "-Wall", "-o", str(OUT), str(SRC), "-lm"]
    subprocess.run(cmd, check=True)
    return OUT


if __name__ == "__main__":
    print(build())
