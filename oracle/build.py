"""Build the oracle's C restatement (test infrastructure) into oracle/libhkv_oracle.so.

    python oracle/build.py
"""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "hkv_oracle.c")
OUT = os.path.join(HERE, "libhkv_oracle.so")

CFLAGS = ["-O2", "-fPIC", "-shared", "-std=c11", "-ffp-contract=off", "-fno-fast-math",
          "-msse2", "-mfpmath=sse", "-Wall", "-Wextra"]


def build(verbose=True):
    tmp = OUT + ".tmp"
    cmd = ["gcc"] + CFLAGS + ["-o", tmp, SRC, "-lm"]
    if verbose:
        print("[oracle] " + " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build())
