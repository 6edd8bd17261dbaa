"""The CPU suite's host code under AddressSanitizer and
UndefinedBehaviorSanitizer: the oracle (oracle/moe_oracle.c, built by gcc
with -fsanitize=address,undefined) runs the oracle tests, and the library's
safetensors reader (st.hip's host code, built host-only by hipcc with clang's
sanitizers) runs the safetensors tests, including its malformed-header cases.
Each suite runs in a child process with the sanitizer runtime preloaded
(tests/asan/Makefile); any report aborts the child and fails the test."""
import os
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
ASAN = os.path.join(HERE, "asan")


def build():
    subprocess.run(["make", "-s", "-C", ASAN, "all"], check=True, capture_output=True)


def run_under(runtime, env_extra, test_file, k=None):
    env = dict(os.environ)
    pre = env.get("LD_PRELOAD")
    env["LD_PRELOAD"] = runtime + (":" + pre if pre else "")
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=1:halt_on_error=1"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    env.update(env_extra)
    # the runtime is really in the child, and the sanitized library loads under it
    probe = ("import ctypes, os; maps = open('/proc/self/maps').read(); "
             "assert 'asan' in maps, 'no sanitizer runtime mapped'; "
             "ctypes.CDLL(os.environ.get('RMDA_ORACLE_LIB') or os.environ['RMDA_MOE_PARTIAL_LIB']); print('probe ok')")
    r = subprocess.run([sys.executable, "-c", probe], env=env, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "probe ok" in r.stdout, (r.stdout + r.stderr)[-2000:]
    cmd = [sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider", "-m", "not gpu",
           os.path.join(HERE, test_file)]
    if k:
        cmd += ["-k", k]
    r = subprocess.run(cmd, cwd=REPO, env=env, capture_output=True, text=True, timeout=900)
    tail = (r.stdout + r.stderr)[-3000:]
    assert r.returncode == 0, tail
    assert "ERROR: AddressSanitizer" not in r.stderr and "runtime error:" not in r.stderr, tail
    return r.stdout


def gcc_runtime(name):
    p = subprocess.run(["gcc", "-print-file-name=" + name], capture_output=True, text=True).stdout.strip()
    if not os.path.isabs(p) or not os.path.exists(p):
        pytest.skip("%s not available" % name)
    return p


def clang_asan_runtime():
    import glob
    hits = sorted(glob.glob("/opt/rocm/lib/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not hits:
        pytest.skip("clang's AddressSanitizer runtime not available")
    return hits[-1]


def test_oracle_under_sanitizers():
    build()
    rt = gcc_runtime("libasan.so") + ":" + gcc_runtime("libubsan.so")
    out = run_under(rt, {"RMDA_ORACLE_LIB": os.path.join(ASAN, "_build", "libmoe_oracle.so")},
                    "test_cpu_oracle.py")
    assert "passed" in out


def test_safetensors_reader_under_sanitizers():
    build()
    out = run_under(clang_asan_runtime(), {"RMDA_MOE_PARTIAL_LIB": os.path.join(ASAN, "_build", "librmda_st.so")},
                    "test_cpu_safetensors.py")
    assert "passed" in out
