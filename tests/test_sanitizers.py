"""The host-side C code under AddressSanitizer and UndefinedBehaviorSanitizer:
the oracle (oracle/qwn_oracle.c, oracle/qwn_oracle_decoder.c), the host
decoder with its ABI loader (qwanto_amd/host/qwn_host_decoder.c) and the fake
qwn_cuda.so it loads, all rebuilt with -fsanitize=address,undefined
-fno-sanitize-recover=all, then the CPU tests that drive them (oracle kernels
against the reference's golden vectors, the oracle decoder against the
reference decoder, every loader branch and the host decoder end to end over
the computing fake) run in a child Python with the ASan runtime preloaded.
Any report aborts the child.  A planted heap overflow and a planted signed
overflow, built and run the same way, show that the set-up reports at all."""
import os
import shutil
import subprocess
import sys

import pytest

from qwanto_amd import build

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN_CFLAGS = "-fsanitize=address,undefined -fno-sanitize-recover=all -fno-omit-frame-pointer"
SUITE = ["tests/test_oracle.py", "tests/test_decoder_oracle.py", "tests/test_loader_branches.py"]

PLANTED = r"""
#include <stdlib.h>
int heap_overflow(int n) {
    int *p = (int *)malloc(sizeof(int) * (size_t)n);
    for (int i = 0; i < n; i++) p[i] = i;
    volatile int v = p[n];          /* one past the end */
    free(p);
    return v;
}
int signed_overflow(int x) { return x + 2147483647; }
"""


def _asan_runtime() -> str:
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc absent")
    path = subprocess.run([gcc, "-print-file-name=libasan.so"], capture_output=True, text=True,
                          check=True).stdout.strip()
    if not os.path.isabs(path) or not os.path.exists(path):
        pytest.skip("no ASan runtime next to gcc")
    return path


@pytest.fixture(scope="module")
def san_env(tmp_path_factory):
    runtime = _asan_runtime()
    out = tmp_path_factory.mktemp("san")
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "sanitize", f"SAN_DIR={out}"], check=True)
    host = build.build_host_decoder(out=str(out / "libqwn_host_decoder.so"), sanitize=True)
    env = dict(os.environ, LD_PRELOAD=runtime, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1", QWN_ORACLE_LIB=str(out / "liboracle.so"),
               QWN_HOST_DECODER_LIB=host, QWN_FAKE_CFLAGS=SAN_CFLAGS)
    return out, env


def test_cpu_suite_under_sanitizers(san_env):
    _, env = san_env
    r = subprocess.run([sys.executable, "-m", "pytest", *SUITE, "-q", "-x", "-m", "not gpu",
                        "-p", "no:cacheprovider"], cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    text = r.stdout + r.stderr
    assert r.returncode == 0, text[-4000:]
    assert "AddressSanitizer" not in text and "runtime error:" not in text, text[-4000:]
    assert " passed" in text


@pytest.mark.parametrize("call,report", [("heap_overflow(4)", "heap-buffer-overflow"),
                                         ("signed_overflow(5)", "runtime error: signed integer overflow")])
def test_planted_mistakes_are_reported(san_env, call, report):
    out, env = san_env
    src, lib = out / "planted.c", out / "libplanted.so"
    if not lib.exists():
        src.write_text(PLANTED)
        subprocess.run(["gcc", "-O1", "-shared", "-fPIC", *SAN_CFLAGS.split(), str(src), "-o", str(lib)],
                       check=True)
    code = f"import ctypes; ctypes.CDLL({str(lib)!r}).{call}"
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=120)
    assert r.returncode != 0
    assert report in r.stderr, r.stderr[-2000:]
