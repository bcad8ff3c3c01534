"""Compiles the oracle's C replica (ordered.c) with gcc into oracle/_build/.
Test infrastructure only."""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
SO = os.path.join(HERE, "_build", "liboracle_ordered.so")


def build():
    os.makedirs(os.path.dirname(SO), exist_ok=True)
    tmp = SO + ".tmp"
    cmd = ["gcc", "-O2", "-fopenmp", "-ffp-contract=off", "-fno-fast-math", "-shared", "-fPIC",
           os.path.join(HERE, "ordered.c"), "-o", tmp, "-lm"]
    subprocess.run(cmd, check=True)
    os.replace(tmp, SO)
    return SO


if __name__ == "__main__":
    print(build())
