"""Build recipe for the CPU oracle (test infrastructure only).

Compiles ``oracle/mis_oracle.c`` into ``oracle/_build/libmis_oracle.so`` with
gcc.  No fast-math and no FP contraction, so every float operation in the
restatement is a single IEEE binary32/binary64/x87 operation.
"""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(OUT_DIR, "libmis_oracle.so")


def build_oracle(verbose: bool = False) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    src = os.path.join(HERE, "mis_oracle.c")
    tmp = LIB + ".tmp"
    cmd = ["gcc", "-O2", "-fopenmp", "-fPIC", "-shared", "-fno-fast-math",
           "-ffp-contract=off", "-std=c11", "-Wall", "-o", tmp, src, "-lm"]
    if verbose:
        print(" ".join(cmd))
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build_oracle(verbose=True))
