"""Builds the gfx950 library indecis_amd/libindecis_hip.so with hipcc.

Every source is compiled for gfx950 only, with -ffp-contract=off (the
kernels round exactly where the reference rounds) and packed FP32 ops
disabled.
"""
import concurrent.futures as cf
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
SO = os.path.join(HERE, "libindecis_hip.so")
SOURCES = ["gemm_i8.hip", "gemm_as.hip", "gemm_ws.hip", "gemm_res.hip", "mlp_res.hip", "mlp_block.hip", "qkv_attn.hip", "rownorm.hip", "attention_i8.hip", "outliers.hip", "safetensors.cpp", "tokenizer.cpp", "embed.cpp", "host_sched.cpp", "ixh_api.cpp"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "-x", "hip", "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off", "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


# Per-source flags. attention_i8.hip: MFMA results in VGPRs, so the score
# tiles feed the VALU softmax without v_accvgpr_read moves (same register
# total, same occupancy).
EXTRA = {"attention_i8.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}


def _compile(src, verbose):
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [HIPCC, *FLAGS, *EXTRA.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{err}")
    if verbose and err.strip():
        print(err, flush=True)
    return obj


def build(verbose=False, jobs=4):
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), SOURCES))
    tmp = SO + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, SO)
    return SO


if __name__ == "__main__":
    print(build(verbose=True))
