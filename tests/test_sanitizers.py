"""AddressSanitizer and UndefinedBehaviorSanitizer over the host code: the
scalar oracle (oracle/nerf_oracle.cpp) and the host harness (PNG, zlib,
JSON, dataset loading, PSNR) are rebuilt with -fsanitize=address,undefined
(g++, host code only) and their CPU test files run against those builds in
a child process with the ASan runtime preloaded.  Any sanitizer report
fails the child (-fno-sanitize-recover=undefined; ASan aborts on the first
error)."""
import os
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
TESTS = ["tests/test_oracle_fp16.py", "tests/test_oracle_rng.py", "tests/test_oracle_hashgrid.py", "tests/test_oracle_mlp_sh.py", "tests/test_oracle_march_composite.py", "tests/test_oracle_train.py",
         "tests/test_oracle_train_rays.py", "tests/test_oracle_scene.py", "tests/test_oracle_cascades.py", "tests/test_oracle_refmodel.py", "tests/test_oracle_uniform.py", "tests/test_harness.py"]


def _runtime(name: str) -> str:
    out = subprocess.run(["g++", f"-print-file-name={name}"], capture_output=True, text=True, check=True).stdout.strip()
    return out if os.path.sep in out and Path(out).exists() else ""


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ is required for the sanitizer builds")
def test_oracle_and_harness_under_asan_ubsan(tmp_path):
    asan = _runtime("libasan.so")
    if not asan:
        pytest.skip("g++ has no AddressSanitizer runtime here")
    subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "sanitize"], check=True)
    sys.path.insert(0, str(ROOT))
    from nerf_amd import build as nb

    host = nb.build_harness_sanitized(tmp_path / "host")
    env = dict(os.environ, LD_PRELOAD=asan, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1", UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1",
               NERF_ORACLE_LIB=str(ROOT / "oracle" / "_san" / "liboracle.so"), NERF_HOST_LIB=str(host))
    proc = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-m", "not gpu", "-p", "no:cacheprovider", *TESTS], cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    out = proc.stdout + proc.stderr
    assert proc.returncode == 0, out[-4000:]
    assert "runtime error" not in out and "AddressSanitizer" not in out, out[-4000:]
    assert " passed" in out
