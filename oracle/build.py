"""Build recipe for the oracle's C restatement (test infrastructure only):
`gcc -O2 -ffp-contract=off -shared` of oracle/csrc/oracle.c into
oracle/liboracle.so (git-ignored; it travels with the tree like every built
library). The reference itself is Python with Trainium-only device code, so
there is no reference build (no oracle/_ref)."""

from __future__ import annotations

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "csrc" / "oracle.c"
LIB = HERE / "liboracle.so"


def build() -> Path:
    cmd = ["gcc", "-O2", "-ffp-contract=off", "-fPIC", "-shared", str(SRC), "-o", str(LIB), "-lm"]
    subprocess.run(cmd, check=True)
    return LIB


if __name__ == "__main__":
    print(build())
