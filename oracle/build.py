"""Build the CPU oracle library (test infrastructure only).

Compiles oracle/peco_oracle.c with gcc into oracle/_build/libpeco_oracle.so.
No part of the reference is compiled here: the reference path is Python/torch
(plus CUDA kernels that need nvcc and an NVIDIA GPU), so there is no reference
build under oracle/_ref.
"""
import os
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
SOURCE = HERE / "peco_oracle.c"
OUTPUT = HERE / "_build" / "libpeco_oracle.so"

FLAGS = ["-O3", "-march=x86-64-v3", "-ffp-contract=off", "-fno-fast-math", "-fopenmp",
         "-shared", "-fPIC", "-std=c11"]


def build(force: bool = False) -> Path:
    OUTPUT.parent.mkdir(exist_ok=True)
    if not force and OUTPUT.exists() and OUTPUT.stat().st_mtime_ns >= SOURCE.stat().st_mtime_ns:
        return OUTPUT
    tmp = OUTPUT.with_suffix(f".{os.getpid()}.tmp")
    cmd = [os.environ.get("CC", "gcc"), *FLAGS, str(SOURCE), "-o", str(tmp), "-lm"]
    subprocess.run(cmd, check=True)
    os.replace(tmp, OUTPUT)
    return OUTPUT


if __name__ == "__main__":
    print(build(force=True))
