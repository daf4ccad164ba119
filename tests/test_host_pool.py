"""The host thread pool under back-to-back jobs, with more threads than cores.

Builds tests/host_pool_stress.cpp against the pool's source with ThreadSanitizer and with
AddressSanitizer (host code only, g++) and runs it: every unit of every job must run
exactly once, inside its own job, with no data race and no access to a finished job's
storage.
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HOST = os.path.join(ROOT, "redukt_amd", "csrc", "host")


@pytest.mark.parametrize("sanitizer,jobs", [("thread", 3000), ("address", 20000)])
def test_pool_back_to_back_jobs(tmp_path, sanitizer, jobs):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    exe = str(tmp_path / f"stress_{sanitizer}")
    cmd = ["g++", "-std=c++17", "-O1", "-g", f"-fsanitize={sanitizer}", "-pthread", f"-I{HOST}",
           os.path.join(ROOT, "tests", "host_pool_stress.cpp"), os.path.join(HOST, "host_pool.cpp"), "-o", exe]
    subprocess.run(cmd, check=True)
    env = dict(os.environ, REDUKT_HOST_THREADS="24", TSAN_OPTIONS="halt_on_error=1",
               ASAN_OPTIONS="detect_leaks=0")
    r = subprocess.run([exe, str(jobs)], env=env, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-4000:]
    assert r.stdout.startswith("ok:"), r.stdout
