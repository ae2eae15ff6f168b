"""Builds the CPU oracle (test infrastructure only) into oracle/liboracle.so.

The reference (Go 1.27 + GOEXPERIMENT=simd + Go assembly) cannot be built
in this image: there is no Go toolchain, so there is no oracle/_ref build.
The oracle is the C restatement in indecis_oracle.c; vnni.c adds the
VPDPBUSD-tiled GEMM the timed CPU baseline uses (same bits).
"""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
SO = os.path.join(HERE, "liboracle.so")

# -ffp-contract=off: no implicit fused multiply-add, every rounding where
# the reference rounds. x86-64-v3 (AVX2+FMA) runs on every MI355X host.
CFLAGS = ["-O3", "-march=x86-64-v3", "-ffp-contract=off", "-fno-fast-math",
          "-fopenmp", "-fPIC", "-shared", "-std=c11", "-Wall"]


def build(verbose=False):
    srcs = [os.path.join(HERE, f) for f in ("indecis_oracle.c", "vnni.c")]
    tmp = SO + ".tmp"
    cmd = ["gcc", *CFLAGS, *srcs, "-o", tmp, "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, SO)
    return SO


if __name__ == "__main__":
    print(build(verbose=True))
