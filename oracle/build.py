"""Builds the CPU oracle (test infrastructure): oracle/_build/libud_oracle.so from ud_oracle.c.

The reference implementation of this path is Swift + Metal and cannot be compiled here, so there
is no oracle/_ref build; the oracle is this plain-C restatement.
"""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(OUT_DIR, "libud_oracle.so")


def build(verbose=False):
    os.makedirs(OUT_DIR, exist_ok=True)
    tmp = LIB + ".tmp"
    cmd = ["gcc", "-O3", "-std=c11", "-mavx2", "-mfma", "-fopenmp", "-fPIC", "-shared",
           "-fvisibility=hidden", os.path.join(HERE, "ud_oracle.c"), "-o", tmp, "-lm"]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError("oracle build failed:\n" + r.stdout)
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
