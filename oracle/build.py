"""Build the CPU oracle (test infrastructure) -> oracle/liborc.so with gcc.

The reference implementation of this path is Objective-C++ over Metal and MLX
(core/kernels/primitives/q_gemm_dequant_primitive.mm includes Metal/Metal.hpp and
mlx/backend/metal/device.h); it cannot be compiled here, so there is no oracle/_ref.
"""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liborc.so")


def build():
    cmd = ["gcc", "-O2", "-fopenmp", "-ffp-contract=off", "-fPIC", "-shared", "-std=c11",
           "-Wall", os.path.join(HERE, "orc.c"), "-o", LIB, "-lm"]
    subprocess.run(cmd, check=True)
    return LIB


if __name__ == "__main__":
    print(build())
