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
    ("mq_encoder.hip", []),
    ("mq_bert.cpp", ["-x", "hip"]),
    ("mq_decoder.hip", []),
    ("mq_decoder_run.cpp", ["-x", "hip"]),
    ("mq_gguf.cpp", ["-x", "hip"]),
    ("mq_gguf_load.cpp", ["-x", "hip"]),
    ("mq_ops.hip", ["-ffp-contract=off"]),
]
# The backend compiles against ggml's backend headers.  Standalone builds use the
# compat transcription in csrc/ggml_compat (and libggml-compat.so for the ggml
# symbols); an integration sets MQ_GGML_INCLUDE to ggml's include+src dirs and
# links the backend against ggml instead.
GGML_INC = os.environ.get("MQ_GGML_INCLUDE", os.path.join(CSRC, "ggml_compat")).split(os.pathsep)
GGML_SOURCES = [
    ("ggml_backend_mi355.cpp", ["-x", "hip", *[f"-I{d}" for d in GGML_INC if d]]),
]
COMPAT_SOURCES = [
    ("ggml_compat/ggml_compat.cpp", ["-x", "c++", "-I", os.path.join(CSRC, "ggml_compat")]),
]

LIBMQ = os.path.join(HERE, "libmq.so")
LIBGGML = os.path.join(HERE, "libggml-mi355.so")
LIBCOMPAT = os.path.join(HERE, "libggml-compat.so")
BIN = os.path.join(HERE, "bin")
TESTS = os.path.join(ROOT, "tests")


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


def build_test_driver():
    """tests/native/*.cpp -> crispembed_amd/bin/ (test code: test-backend-mi355 links the CPU
    oracle as the checker; test-bert-graph-mi355 writes its result for the Python test to check)."""
    os.makedirs(BIN, exist_ok=True)
    oracle = os.path.join(ROOT, "oracle")
    common = ["-O2", "-std=c++17", "-I", os.path.join(CSRC, "ggml_compat"), "-I", os.path.join(ROOT, "include"),
              "-I", oracle]
    libs = ["-L", HERE, "-lggml-mi355", "-lggml-compat", "-lmq", "-Wl,-rpath," + HERE, "-Wl,-rpath,$ORIGIN/.."]
    outs = []
    with_oracle = ["-L", oracle, "-loracle", "-Wl,-rpath," + oracle, "-Wl,-rpath,$ORIGIN/../../oracle"]
    rocm = os.path.dirname(os.path.dirname(os.path.realpath(HIPCC)))
    with_hip = ["-I", os.path.join(rocm, "include"), "-D__HIP_PLATFORM_AMD__", "-L", os.path.join(rocm, "lib"),
                "-lamdhip64", "-Wl,-rpath," + os.path.join(rocm, "lib")]
    for src, name, extra in (("test_backend_mi355.cpp", "test-backend-mi355", with_oracle),
                             ("test_bert_graph_mi355.cpp", "test-bert-graph-mi355", []),
                             ("test_decoder_graph_mi355.cpp", "test-decoder-graph-mi355", with_oracle + with_hip)):
        out = os.path.join(BIN, name)
        cmd = ["g++", *common, os.path.join(TESTS, "native", src), "-o", out + ".tmp", *libs, *extra]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"driver build failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
        os.replace(out + ".tmp", out)
        outs.append(out)
    return outs


# Host-side AddressSanitizer + UndefinedBehaviorSanitizer build of the same libraries, for the
# CPU tests (GGUF reader and loaders, host quantizer, C ABI argument checks): every host
# translation unit instrumented, device code built as usual but never run (the CPU tests launch
# no kernel).  The shared libraries leave the sanitizer runtime unresolved; the test process
# preloads clang's (asan_runtime()), which also carries the UBSan handlers.
ASAN_DIR = os.path.join(HERE, "_asan")
SAN_FLAGS = ("-O1 -g -Xarch_host -fsanitize=address -Xarch_host -fsanitize=undefined "
             "-Xarch_host -fno-sanitize-recover=undefined -Xarch_host -fno-omit-frame-pointer").split()


def asan_runtime():
    """clang's shared ASan runtime (the compiler that built the sanitized libraries)."""
    clang = os.path.join(os.path.dirname(os.path.realpath(HIPCC)), "..", "llvm", "bin", "clang")
    r = subprocess.run([clang, "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True)
    path = r.stdout.strip()
    return path if r.returncode == 0 and os.path.isabs(path) and os.path.exists(path) else None


def build_sanitized(verbose=True):
    bdir = os.path.join(ASAN_DIR, "obj")
    os.makedirs(bdir, exist_ok=True)

    def comp(src, extra):
        common = [f for f in COMMON if f != "-O3"]
        obj = os.path.join(bdir, src.replace("/", "_") + ".o")
        cmd = [HIPCC, *common, *SAN_FLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
        return obj

    srcs = list(MQ_SOURCES) + list(GGML_SOURCES) + list(COMPAT_SOURCES)
    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 4)) as ex:
        objs = list(ex.map(lambda a: comp(*a), srcs))
    n = len(MQ_SOURCES)
    lib_mq, lib_ggml, lib_compat = (os.path.join(ASAN_DIR, x) for x in ("libmq.so", "libggml-mi355.so",
                                                                          "libggml-compat.so"))
    _link(objs[:n], lib_mq)
    _link(objs[n + len(GGML_SOURCES):], lib_compat)
    _link(objs[n:n + len(GGML_SOURCES)], lib_ggml, ["-L", ASAN_DIR, "-lmq", "-lggml-compat", "-Wl,-rpath,$ORIGIN"])
    r = subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "asan"], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"sanitized oracle build failed:\n{r.stdout}\n{r.stderr}")
    if verbose:
        print(f"built the host-sanitized libraries in {ASAN_DIR} and oracle/_asan")
    return ASAN_DIR


def build(verbose=True):
    os.makedirs(BUILD, exist_ok=True)
    srcs = list(MQ_SOURCES) + list(GGML_SOURCES)
    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 4)) as ex:
        objs = list(ex.map(lambda a: _compile(*a), srcs))
        compat_objs = list(ex.map(lambda a: _compile(*a), COMPAT_SOURCES))
    mq_objs = objs[: len(MQ_SOURCES)]
    _link(mq_objs, LIBMQ)
    _link(compat_objs, LIBCOMPAT)
    _link(objs[len(MQ_SOURCES):], LIBGGML, ["-L", HERE, "-lmq", "-lggml-compat", "-Wl,-rpath,$ORIGIN"])
    if verbose:
        print(f"built {LIBMQ}, {LIBGGML}, {LIBCOMPAT}")
    return LIBMQ


if __name__ == "__main__":
    build()
    if os.path.exists(os.path.join(ROOT, "oracle", "liboracle.so")):
        build_test_driver()
    sys.exit(0)
