"""Builds the native libraries in-tree (they travel to the GPU box with the source tree):

  malkin_amd/libmalkin_hip.so    gfx950 kernels + C ABI (include/malkin_hip.h, include/malkin_model.h) + host model
  malkin_amd/libmalkin_synth.so  deterministic synthetic GGUF writer (host only)

Every HIP translation unit is compiled with -ffp-contract=off (bit-exact fp32 chains: every fused multiply-add is an
explicit fmaf) and without packed-FP32 instructions.
"""
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
BUILD = os.path.join(HERE, "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("MALKIN_ARCH", "gfx950")

HIP_SOURCES = [
    "csrc/kernels/pack.hip",
    "csrc/kernels/gemv.hip",
    "csrc/kernels/gemv_mma.hip",
    "csrc/kernels/gemm.hip",
    "csrc/kernels/gemm_kq.hip",
    "csrc/kernels/quant.hip",
    "csrc/kernels/attn.hip",
    "csrc/kernels/decode.hip",
    "csrc/kernels/cut.hip",
    "csrc/kernels/rowpath.hip",
    "csrc/kernels/sample.hip",
    "csrc/kernels/capi.cpp",
    "csrc/host/gguf.cpp",
    "csrc/host/model.cpp",
    "csrc/host/sampler.cpp",
    "csrc/host/engine.cpp",
    "csrc/host/capi_model.cpp",
    "csrc/server/json.cpp",
    "csrc/server/http.cpp",
    "csrc/server/server.cpp",
]

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++20", "-fPIC", "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt", "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # The first kernel arguments arrive in SGPRs at wave launch instead of through a scalar load of the kernarg
    # segment: one memory round trip less at the start of every kernel (all of them are latency-exposed there).
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable", "-Wno-unused-but-set-variable",
    f"-I{ROOT}/include",
]

# Per-source extra flags. gemm.hip: MFMA results in ordinary VGPRs (its epilogue reads every accumulator element
# with VALU instructions; the AGPR form would add one v_accvgpr_read per element and block).
EXTRA_FLAGS = {
    "csrc/kernels/gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    "csrc/kernels/gemm_kq.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}

LIB = os.path.join(HERE, "libmalkin_hip.so")
SYNTH = os.path.join(HERE, "libmalkin_synth.so")


def _run(cmd):
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in p.stdout.splitlines() if "packed-fp32-ops" not in l)
    if p.returncode != 0:
        raise RuntimeError(f"command failed ({p.returncode}): {' '.join(cmd)}\n{out}")
    return out


def _obj(src):
    return os.path.join(BUILD, src.replace("/", "_").rsplit(".", 1)[0] + ".o")


def build_hip(jobs=None, verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    srcs = [s for s in HIP_SOURCES if os.path.exists(os.path.join(HERE, s))]

    def compile_one(s):
        lang = ["-x", "hip"] if s.endswith(".hip") else []
        cmd = [HIPCC] + HIP_FLAGS + EXTRA_FLAGS.get(s, []) + lang + ["-c", os.path.join(HERE, s), "-o", _obj(s)]
        out = _run(cmd)
        if verbose and out.strip():
            print(out)
        return s

    with cf.ThreadPoolExecutor(max_workers=jobs or min(8, os.cpu_count() or 1)) as ex:
        list(ex.map(compile_one, srcs))
    tmp = LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-pthread", "-o", tmp] + [_obj(s) for s in srcs])
    os.replace(tmp, LIB)
    return LIB


def build_synth():
    src = os.path.join(HERE, "synth", "synth_gguf.c")
    tmp = SYNTH + ".tmp"
    _run(["gcc", "-std=c11", "-O2", "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-shared", "-pthread", "-Wall",
          "-o", tmp, src])
    os.replace(tmp, SYNTH)
    return SYNTH


def build_all(verbose=False):
    build_synth()
    build_hip(verbose=verbose)


if __name__ == "__main__":
    build_all(verbose="-v" in sys.argv)
    print("built", LIB, SYNTH)
