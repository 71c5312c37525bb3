"""Runs libdpep's kernel source on the CPU (tests/emu): every kernel of a
step, one std::thread per GPU thread, under AddressSanitizer with exact-size
buffers and a poisoned LDS tail, compared with the float64 oracle.  Catches
out-of-bounds indexing, cross-wave races (threads really run concurrently)
and transform mistakes without a GPU.  Each case runs two steps and checks
that the side map and strip flags are left clean for the next step."""
import os
import shutil
import subprocess

import pytest

from conftest import ROOT

CLANG = "/opt/rocm/llvm/bin/clang++"
CLANGC = "/opt/rocm/llvm/bin/clang"


@pytest.fixture(scope="module")
def emu(tmp_path_factory):
    if not os.path.exists(CLANG):
        pytest.skip("ROCm clang++ not available")
    d = tmp_path_factory.mktemp("emu")
    obj = d / "oracle.o"
    subprocess.run([CLANGC, "-O1", "-g", "-fsanitize=address", "-c",
                    os.path.join(ROOT, "oracle", "dpep_oracle.c"), "-o", str(obj)],
                   check=True)
    exe = d / "emu_main"
    subprocess.run([CLANG, "-std=c++20", "-O1", "-g", "-fsanitize=address",
                    "-fno-omit-frame-pointer",
                    "-I", os.path.join(ROOT, "tests", "emu"),
                    "-I", os.path.join(ROOT, "dreamplacett-framework_amd", "csrc"),
                    "-I", os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "tests", "emu", "emu_main.cpp"), str(obj),
                    "-o", str(exe), "-lpthread", "-lm"], check=True)
    return str(exe)


# ch=<n> forces n entries per strip work item (exercises the split-strip
# reduce); tall gives a tenth of the cells a span of 3..40 rows (side map B);
# stage forces K3's staged form (the library picks it from 512 strips on);
# off moves the die's lower-left corner off the origin.
CASES = [
    "f32 8 8 50", "f32 16 16 200 tall", "f32 8 32 60 nopot", "f32 16 128 3000 ch=128",
    "f32 128 16 300", "f64 8 8 40", "f64 64 64 1000 ch=100 tall",
    "f32 64 64 2000 ch=64 tall", "f32 256 32 600", "f32 32 256 400 tall",
    "f32 32 2048 500", "f64 32 2048 300 tall",
    "f32 32 2048 0",         # no cells: the last kernel runs the potential alone
    "f32 32 2048 400 nopot",
    "f32 16 4096 2000 tall", "f64 16 4096 100",
    "f32 16 128 9000 tall",  # chunks chosen per step: both strips split
    "f32 8 8192 3000 tall",  # 2-row strips, the largest LDS tile and row FFT
    "f32 64 64 2000 tall stage", "f64 64 64 1500 ch=100 stage",
    "f32 16 128 9000 tall stage",  # blocks beyond the stage: records stored straight
    # one-pass blocks of 4 and 5 cells per thread (three blocks per "CU" of the
    # 2-CU emulated device at float32, two at float64), and past 5 cells per
    # thread the 2048-cell blocks in rounds, with tall cells
    "f32 64 64 10800", "f32 64 64 13200 tall", "f32 64 64 16800 tall",
    "f64 64 64 7200", "f64 64 64 8800 tall",
    "f32 64 64 3000 tall off", "f64 16 128 2000 off",
]


@pytest.mark.parametrize("case", CASES)
def test_kernels_in_bounds_and_accurate(emu, case):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1")
    r = subprocess.run([emu] + case.split(), capture_output=True, text=True,
                       timeout=600, env=env)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "emu " in r.stdout


# The spectral passes alone at every FFT length from 8 to 8192 on either axis
# (the column pass at 2048 and 4096 rows holds 210-229 VGPRs' worth of state,
# 8192 the largest LDS use), against the oracle's FFT solve of the same density.
SPECTRAL = ["f32 2048 16", "f32 4096 32", "f32 16 2048", "f32 32 4096", "f32 8192 8",
            "f32 8 8192", "f32 1024 64", "f64 2048 16", "f64 4096 32", "f64 1024 64",
            "f64 16 2048", "f64 32 4096",
            # square grids: the passes with their tile extents compiled in
            "f32 512 512", "f64 512 512", "f32 1024 1024"]


@pytest.mark.parametrize("case", SPECTRAL)
def test_spectral_passes_in_bounds_and_accurate(emu, case):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1")
    r = subprocess.run([emu, "spectral"] + case.split(), capture_output=True, text=True,
                       timeout=600, env=env)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "emu spectral " in r.stdout


def test_float32_record_word(emu):
    """rec_geo / rec_put / rec_view round trip: random cells, the second-strip
    copy of a cell spanning two strips, and cells whose stretched corner lies
    below the die's lower x or y edge decode to the encoded geometry (first
    row and column, offsets within 2^-23 of a bin, extents, area ratio, row
    and column counts reaching the far edge)."""
    r = subprocess.run([emu, "records"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "records ok" in r.stdout


def test_cell_blocks_host_logic(emu):
    """once_blocks / set_count_blocks / count_cells: every cell in exactly one
    one-pass block and one counting part, no part straddling two blocks, the
    kernels' cells-per-thread limits and the cnt rows respected."""
    r = subprocess.run([emu, "blocks"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "blocks ok" in r.stdout
