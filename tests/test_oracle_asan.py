"""The CPU oracle built with AddressSanitizer and UndefinedBehaviorSanitizer
(host code only) and run over every entry point on small ragged shapes, with
each tensor allocated at its exact size (tests/asan/oracle_asan.c)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_oracle_under_asan_ubsan(tmp_path):
    exe = tmp_path / "oracle_asan"
    src = [os.path.join(ROOT, "oracle", f) for f in ("oracle_ops.c", "oracle_model.c")]
    cmd = ["gcc", "-std=c11", "-O1", "-g", "-fopenmp", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=undefined", "-o", str(exe), os.path.join(HERE, "asan", "oracle_asan.c"), *src,
           "-lm", "-ldl"]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    env.pop("LD_PRELOAD", None)
    r = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "clean" in r.stdout
