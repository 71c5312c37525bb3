"""CPU: the shm server's host copy pool (csrc/dpep_copy_pool.h) under
ThreadSanitizer.  The server copies the positions into page-locked staging
before every upload, and the outputs into the shm file before DONE, through
this pool (the reference's ordering: host/density_scatter_ttnn_server_host.cpp
:1335-1349, :1785-1815); a worker left inside an old round while the next
round rebuilds the piece list would let copy() return early.

tests/copy_pool_stress.cpp runs 1e5 copy() rounds of random piece counts with
workers held up at random (yields and sleeps after waking and before pieces),
checks every destination byte after each round, and exits non-zero on a wrong
byte; TSAN (halt_on_error) makes any data race fail the run too."""
import os
import shutil
import subprocess

import pytest

from conftest import PKG

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def stress_bin(tmp_path_factory):
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("g++ not found")
    out = tmp_path_factory.mktemp("copy_pool") / "copy_pool_stress"
    cmd = [cxx, "-std=c++17", "-O1", "-g", "-fsanitize=thread",
           "-I", os.path.join(PKG, "csrc"),
           os.path.join(HERE, "copy_pool_stress.cpp"), "-o", str(out), "-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return str(out)


def test_copy_pool_rounds_are_race_free(stress_bin):
    env = dict(os.environ, TSAN_OPTIONS="halt_on_error=1 exitcode=66")
    r = subprocess.run([stress_bin, "100000", "7"], capture_output=True, text=True,
                       timeout=600, env=env)
    print(r.stdout, r.stderr[-4000:], flush=True)
    assert "ThreadSanitizer" not in r.stderr
    assert r.returncode == 0
    assert "copy_pool_stress ok: 100000 rounds" in r.stdout
