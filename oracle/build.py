"""Build the C restatement of the oracle (``oracle/libqmm_oracle.so``).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  The reference has no
C/C++ source on this path (its kernels are Metal strings inside Python, and
the arithmetic lives in the un-vendored mlx==0.32.2), so there is no
``oracle/_ref`` build; this library is the project's own restatement.
"""

from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "qmm_oracle.c")
OUT = os.path.join(HERE, "libqmm_oracle.so")


def build() -> str:
    tmp = OUT + ".tmp"
    cmd = ["gcc", "-O3", "-std=c11", "-fPIC", "-shared", "-fopenmp", "-Wall", "-o", tmp, SRC]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"gcc failed: {res.stderr}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build())
