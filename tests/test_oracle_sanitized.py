"""The CPU oracle under AddressSanitizer and UndefinedBehaviorSanitizer:
tests/cpp/oracle_asan.c calls every exported oracle function on small,
ragged shapes with exact-size buffers (the sizes oracle/__init__.py
allocates), built together with oracle/oracle.c with gcc -fsanitize=address,
undefined.  An out-of-bounds access, use after free or undefined operation
aborts the driver; it also checks a few invariants (probability rows sum to
one, CE gradient rows sum to zero)."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_oracle_memory_safe_under_sanitizers(tmp_path):
    exe = tmp_path / "oracle_asan"
    cmd = ["gcc", "-std=c11", "-O1", "-g", "-fno-omit-frame-pointer", "-ffp-contract=off", "-fopenmp",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           str(ROOT / "oracle" / "oracle.c"), str(ROOT / "tests" / "cpp" / "oracle_asan.c"), "-lm", "-o", str(exe)]
    build = subprocess.run(cmd, capture_output=True, text=True)
    if build.returncode != 0 and "sanitize" in build.stderr:
        pytest.skip("gcc without sanitizer runtimes: " + build.stderr[:200])
    assert build.returncode == 0, build.stderr
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120,
                         env={"ASAN_OPTIONS": "detect_leaks=1:abort_on_error=0", "OMP_NUM_THREADS": "2",
                              "PATH": "/usr/bin:/bin"})
    assert res.returncode == 0, res.stdout[-2000:] + res.stderr[-4000:]
    assert "OK oracle under ASan/UBSan" in res.stdout
