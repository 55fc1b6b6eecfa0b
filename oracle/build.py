"""Builds the CPU oracle (test infrastructure) into oracle/liboracle.so with gcc."""

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
SOURCE = os.path.join(HERE, "inflate_oracle.c")
LIBRARY = os.path.join(HERE, "liboracle.so")


def build():
    tmp = LIBRARY + ".tmp"
    cmd = ["gcc", "-O2", "-std=c11", "-Wall", "-Wextra", "-fPIC", "-shared", SOURCE, "-o", tmp]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode:
        raise RuntimeError("oracle build failed:\n" + proc.stdout + proc.stderr)
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build())
