"""The host code under AddressSanitizer + UndefinedBehaviorSanitizer: the CPU test suite (GGUF
reader with every truncation and malformed-header case, the model loaders' rejections, the host
quantizer, the C ABI's argument checks, the oracle and its pins) run again against the
host-sanitized build of libmq / libggml-mi355 / libggml-compat (crispembed_amd/_asan, built by
crispembed_amd/build.py build_sanitized) and of the oracle (oracle/_asan), with clang's sanitizer
runtime preloaded.  Any invalid access, leak-free use-after-free, or undefined behaviour (signed
overflow, misaligned load, bad shift, invalid enum or bool value) aborts the run.  Leak checking
is off: the Python interpreter itself does not free everything at exit."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ASAN_DIR = os.path.join(ROOT, "crispembed_amd", "_asan")
ORACLE_ASAN = os.path.join(ROOT, "oracle", "_asan", "liboracle.so")
HERE = os.path.basename(__file__)


def _cpu_test_files():
    out = []
    for f in sorted(os.listdir(os.path.dirname(os.path.abspath(__file__)))):
        if not (f.startswith("test_") and f.endswith(".py")) or f == HERE:
            continue
        text = open(os.path.join(os.path.dirname(os.path.abspath(__file__)), f)).read()
        if "pytestmark = pytest.mark.gpu" in text:
            continue
        out.append(os.path.join("tests", f))
    return out


def test_cpu_suite_under_sanitizers():
    sys.path.insert(0, os.path.join(ROOT, "crispembed_amd"))
    import build as B
    rt = B.asan_runtime()
    assert rt, "clang's ASan runtime not found next to hipcc"
    for lib in ("libmq.so", "libggml-mi355.so", "libggml-compat.so"):
        assert os.path.exists(os.path.join(ASAN_DIR, lib)), "run __graft_entry__.build() first"
    assert os.path.exists(ORACLE_ASAN)
    env = dict(os.environ)
    # the runtime must come first; anything already preloaded stays
    env["LD_PRELOAD"] = rt + (":" + env["LD_PRELOAD"] if env.get("LD_PRELOAD") else "")
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=1"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1:halt_on_error=1"
    env["MQ_LIB_DIR"] = ASAN_DIR
    env["MQ_ORACLE_SO"] = ORACLE_ASAN
    env["MQ_SANITIZED_RUN"] = "1"
    files = _cpu_test_files()
    assert len(files) >= 8
    cmd = [sys.executable, "-m", "pytest", "-x", "-q", "-rs", "-m", "not gpu", "-p", "no:cacheprovider",
           f"tests/{HERE}::test_sanitized_build_is_loaded", *files]
    r = subprocess.run(cmd, cwd=ROOT, env=env, capture_output=True, text=True, timeout=1500)
    tail = (r.stdout[-3000:] + r.stderr[-3000:])
    assert r.returncode == 0, tail
    assert " passed" in r.stdout, tail
    assert "runs inside test_cpu_suite_under_sanitizers" not in r.stdout, tail  # the probe ran
    print(r.stdout.strip().splitlines()[-1])


def test_sanitized_build_is_loaded():
    """Inside the sanitized run: the instrumented libraries and the runtime are the ones mapped."""
    if not os.environ.get("MQ_SANITIZED_RUN"):
        pytest.skip("runs inside test_cpu_suite_under_sanitizers")
    import ctypes
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import oracle_ffi as O
    from crispembed_amd import mq
    mq.lib()
    O.Oracle()
    maps = open("/proc/self/maps").read()
    assert os.path.join(ASAN_DIR, "libmq.so") in maps
    assert ORACLE_ASAN in maps
    assert "libclang_rt.asan" in maps
    assert hasattr(ctypes.CDLL(None), "__asan_address_is_poisoned")
