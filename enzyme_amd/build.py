"""Build recipe for libaxon_hip.so (every HIP source under csrc/, gfx950).

Each `csrc/*.hip` file is compiled to an object in `_build/` with hipcc, in
parallel, then linked into `enzyme_amd/lib/libaxon_hip.so`. Per-file extra
flags live in `EXTRA_FLAGS` (the elementwise unit, which holds fused Adam, is built without
FMA contraction so its arithmetic rounds like the fp32 CPU reference).

Run `python -m enzyme_amd.build` (or `__graft_entry__.build()`).
"""

from __future__ import annotations

import hashlib
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = REPO / "include"
BUILD = PKG / "_build"
LIB_DIR = PKG / "lib"
LIB = LIB_DIR / "libaxon_hip.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]

EXTRA_FLAGS: dict[str, list[str]] = {
    "elementwise.hip": ["-ffp-contract=off"],
}


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _headers_digest() -> str:
    h = hashlib.sha256()
    for p in sorted([*CSRC.glob("*.hpp"), *INCLUDE.glob("*.h")]):
        h.update(p.name.encode())
        h.update(p.read_bytes())
    return h.hexdigest()[:16]


def _compile(src: Path, force: bool) -> Path:
    obj = BUILD / (src.stem + ".o")
    flags = COMMON_FLAGS + EXTRA_FLAGS.get(src.name, [])
    stamp = BUILD / (src.stem + ".stamp")
    key = hashlib.sha256(
        src.read_bytes() + " ".join(flags).encode() + _headers_digest().encode()
    ).hexdigest()
    if not force and obj.exists() and stamp.exists() and stamp.read_text() == key:
        return obj
    cmd = [HIPCC, *flags, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(
            f"hipcc failed for {src.name} (exit {proc.returncode}):\n"
            + " ".join(cmd)
            + "\n"
            + proc.stdout
            + proc.stderr
        )
    stamp.write_text(key)
    return obj


def build(force: bool = True, jobs: int | None = None, verbose: bool = True) -> Path:
    """Compile every HIP source and link the shared library. `force=True`
    recompiles every object (the default: a build is always a real build)."""
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    BUILD.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(16, max(1, os.cpu_count() or 1), len(srcs))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(lambda s: _compile(s, force), srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError("link failed:\n" + " ".join(cmd) + "\n" + proc.stdout + proc.stderr)
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} source(s)")
    return LIB


if __name__ == "__main__":
    build(force="--incremental" not in sys.argv)
