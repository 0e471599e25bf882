"""The C oracle under AddressSanitizer + UndefinedBehaviorSanitizer (host
build, `make -C oracle sanitize`): group sizes 4..256, ragged group counts,
NaN / inf / denormal / signed-zero / huge inputs; no memory error, no
undefined behaviour, outputs written within bounds, round-trip ==
quantise + dequantise."""

import os
import shutil
import subprocess

import pytest

ORACLE = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle")


@pytest.mark.skipif(shutil.which("gcc") is None or shutil.which("make") is None,
                    reason="needs gcc and make")
def test_oracle_under_asan_ubsan(tmp_path):
    r = subprocess.run(["make", "-s", "-C", ORACLE, "sanitize", f"SAN_OUT={tmp_path}"],
                       capture_output=True, text=True, timeout=300,
                       env={**os.environ, "ASAN_OPTIONS": "detect_leaks=1:abort_on_error=0",
                            "UBSAN_OPTIONS": "print_stacktrace=1"})
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "sanitized oracle run: ok" in r.stdout
