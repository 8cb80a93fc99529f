"""The oracle under AddressSanitizer and UndefinedBehaviorSanitizer (CPU).

A copy of oracle/c2slm_oracle.c is built with -fsanitize=address,undefined
(the oracle's own floating-point flags kept) and driven through forward,
ingest (rewind, clamp, the max_ctx stop), compute_logits and generate on a
Qwen2 and a Qwen3 model by tests/sanitize_drive.py, in a subprocess with
the sanitizer runtimes preloaded (Python itself is not instrumented).  The
run must be clean; and a copy with one planted out-of-bounds write must be
caught, which shows the instrumentation is live."""
import os
import subprocess
import sys

import pytest

from oracle import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(os.path.dirname(O.__file__), "c2slm_oracle.c")
AVX2_SRC = os.path.join(os.path.dirname(O.__file__), "c2slm_avx2.c")  # the CPU baseline's kernels, linked too
CFLAGS = ["-O1", "-g", "-fPIC", "-std=c11", "-ffp-contract=off", "-fno-fast-math", "-mavx2", "-mfma", "-fopenmp",
          "-fsanitize=address,undefined", "-fno-omit-frame-pointer", "-fno-sanitize-recover=undefined", "-shared"]


def runtime(name: str) -> str:
    p = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True).stdout.strip()
    if not os.path.isabs(p) or not os.path.exists(p):
        pytest.skip(f"{name} not available")
    return p


def build(tmp, text: str) -> str:
    src = tmp / "o.c"
    src.write_text(text)
    so = str(tmp / "liboracle_san.so")
    subprocess.run(["gcc", *CFLAGS, "-o", so, str(src), AVX2_SRC, "-lm"], check=True)
    return so


def drive(so: str, workdir) -> subprocess.CompletedProcess:
    env = dict(os.environ, LD_PRELOAD=f"{runtime('libasan.so')}:{runtime('libubsan.so')}",
               ASAN_OPTIONS="detect_leaks=0", UBSAN_OPTIONS="print_stacktrace=1")
    return subprocess.run([sys.executable, os.path.join(HERE, "sanitize_drive.py"), so, str(workdir)], env=env,
                          capture_output=True, text=True, timeout=600)


def test_oracle_clean_under_asan_and_ubsan(tmp_path):
    r = drive(build(tmp_path, open(SRC).read()), tmp_path)
    assert r.returncode == 0, r.stderr[-3000:]
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr, r.stderr[-3000:]
    assert r.stdout.count(" ok ") == 2


def test_sanitizer_catches_a_planted_overflow(tmp_path):
    text = open(SRC).read()
    old = "for (int i = 0; i < n; ++i) out[i] = (x[i] * inv) * w[i];"
    assert text.count(old) == 1
    r = drive(build(tmp_path, text.replace(old, old.replace("i < n", "i <= n"))), tmp_path)
    assert r.returncode != 0 and "heap-buffer-overflow" in r.stderr
