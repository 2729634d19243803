"""The host half of the C ABI (lithe_amd/csrc/host.cpp: 9-bit packer, .lithe-stream ingest,
status strings) built with g++ under AddressSanitizer + UndefinedBehaviorSanitizer and under
ThreadSanitizer, with tests/native/host_check.cpp as the driver (direct restatements of the
packed residency format, edge sizes, threaded sizes, error paths). CPU only."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SOURCES = [os.path.join(ROOT, "lithe_amd", "csrc", "host.cpp"), os.path.join(ROOT, "tests", "native", "host_check.cpp")]


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
@pytest.mark.parametrize("sanitizers", ["address,undefined", "thread"])
def test_host_code_under_sanitizers(tmp_path, sanitizers):
    exe = tmp_path / "host_check"
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", f"-fsanitize={sanitizers}",
           "-fno-sanitize-recover=all", "-I", os.path.join(ROOT, "include"), *SOURCES, "-o", str(exe), "-pthread"]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1", TSAN_OPTIONS="halt_on_error=1")
    res = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=600)
    if res.returncode != 0 and "does not come first in initial library list" in res.stderr:
        pytest.skip("a preloaded library keeps the sanitizer runtime from loading first in this environment")
    assert res.returncode == 0, res.stderr[-4000:]
    assert "host checks passed" in res.stdout
    assert "Sanitizer" not in res.stderr, res.stderr[-4000:]
