"""Build the CPU oracle library (test infrastructure only).

    python oracle/build.py        -> oracle/build/libds5oracle.so

-ffp-contract=off keeps every a*b+c as a rounded multiply then a rounded add,
as Zig's default (strict) float mode does; -fno-builtin keeps libm calls as
calls. No OpenMP: the reference CPU path is single-threaded.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT_DIR = os.path.join(HERE, "build")
LIB = os.path.join(OUT_DIR, "libds5oracle.so")
SOURCES = [os.path.join(HERE, "ds5_oracle.c")]
CFLAGS = ["-O2", "-std=c11", "-ffp-contract=off", "-fno-fast-math", "-fno-builtin",
          "-fPIC", "-shared", "-Wall", "-Wextra", "-Wno-unused-parameter"]


def build(verbose: bool = False) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    tmp = LIB + ".tmp"
    cmd = ["gcc", *CFLAGS, "-o", tmp, *SOURCES, "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
