"""Exception safety of the host thread pool (csrc/worker_pool.hpp): a task that
throws makes run() rethrow on the calling thread once the run is drained, and
the pool keeps working.  The check is a small C++ program built here with g++
(tests/cpp/worker_pool_check.cpp)."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(HERE), "moe-ascend-opt_amd", "csrc")


def test_pool_rethrows_and_recovers(tmp_path):
    exe = str(tmp_path / "worker_pool_check")
    build = subprocess.run(["g++", "-O2", "-std=c++17", "-pthread", f"-I{CSRC}",
                            os.path.join(HERE, "cpp", "worker_pool_check.cpp"), "-o", exe],
                           stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if build.returncode != 0:
        pytest.fail("build failed:\n" + build.stdout)
    run = subprocess.run([exe], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=120)
    assert run.returncode == 0 and run.stdout.strip() == "ok", run.stdout
