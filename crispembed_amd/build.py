"""Builds libmq.so (the gfx950 kernels + C ABI) and libggml-mi355.so in-tree.

Every HIP translation unit is compiled for gfx950 only.  Flags that matter:
  -Xclang -target-feature -Xclang -packed-fp32-ops   no v_pk_*_f32 instructions
  -fhip-fp32-correctly-rounded-divide-sqrt           IEEE division, as x86 divss
  -ffp-contract=off (quantization / producer files)  no fused multiply-add where
                                                     the result must match ggml's
                                                     CPU rounding bit for bit
"""
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
ROOT = os.path.dirname(HERE)

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
COMMON = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
]
# (source, extra flags)
MQ_SOURCES = [
    ("mq_quant.hip", ["-ffp-contract=off"]),
    ("mq_gemm.hip", []),
    ("mq_gemv.hip", []),
    ("mq_api.cpp", ["-x", "hip"]),
    ("mq_host_quant.cpp", ["-x", "hip", "-ffp-contract=off"]),
]
GGML_SOURCES = [
    ("ggml_backend_mi355.cpp", ["-x", "hip"]),
    ("ggml_compat/ggml_compat.cpp", ["-x", "hip"]),
]

LIBMQ = os.path.join(HERE, "libmq.so")
LIBGGML = os.path.join(HERE, "libggml-mi355.so")


def _compile(src, extra):
    obj = os.path.join(BUILD, src.replace("/", "_") + ".o")
    cmd = [HIPCC, *COMMON, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def _link(objs, out, extra=()):
    tmp = out + ".tmp"
    cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, *extra, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, out)


def build(verbose=True):
    os.makedirs(BUILD, exist_ok=True)
    srcs = list(MQ_SOURCES)
    have_ggml = os.path.exists(os.path.join(CSRC, "ggml_backend_mi355.cpp"))
    if have_ggml:
        srcs += GGML_SOURCES
    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 4)) as ex:
        objs = list(ex.map(lambda a: _compile(*a), srcs))
    mq_objs = objs[: len(MQ_SOURCES)]
    _link(mq_objs, LIBMQ)
    if have_ggml:
        _link(objs[len(MQ_SOURCES):], LIBGGML, ["-L", HERE, "-lmq", "-Wl,-rpath,$ORIGIN"])
    if verbose:
        print(f"built {LIBMQ}" + (f" and {LIBGGML}" if have_ggml else ""))
    return LIBMQ


if __name__ == "__main__":
    build()
    sys.exit(0)
