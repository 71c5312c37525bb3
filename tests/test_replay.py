"""Position-dump replay (dpep.replay): the dump format written by the shm
server's EXPORT_POS_PATH (reference host/density_scatter_ttnn_server_host.cpp
:1686-1726, read by tools/cpu_vs_tt_density.py:12-21)."""
import struct

import numpy as np
import pytest

from dpep import replay


def _dump_bytes(M, N, die, px, py, sx, sy):
    head = struct.pack("<ii", M, N) + struct.pack("<ffff", 0.0, 0.0, die, die) + \
        struct.pack("<i", px.size)
    return head + b"".join(np.asarray(a, "<f4").tobytes() for a in (px, py, sx, sy))


def test_reads_the_reference_layout(tmp_path):
    rng = np.random.default_rng(0)
    px, py, sx, sy = (rng.uniform(0, 100, 37).astype(np.float32) for _ in range(4))
    p = tmp_path / "pos.iter1.bin"
    p.write_bytes(_dump_bytes(64, 32, 640.0, px, py, sx, sy))
    d = replay.read_positions(str(p))
    assert (d.M, d.N, d.nc) == (64, 32, 37) and d.xh == 640.0 and d.yl == 0.0
    for a, b in zip((d.px, d.py, d.sx, d.sy), (px, py, sx, sy)):
        assert np.array_equal(a, b)
    q = tmp_path / "copy.bin"
    replay.write_positions(str(q), d)
    assert q.read_bytes() == p.read_bytes()


def test_rejects_bad_files(tmp_path):
    p = tmp_path / "short.bin"
    p.write_bytes(b"\x00" * 10)
    with pytest.raises(ValueError):
        replay.read_positions(str(p))
    px = np.ones(5, np.float32)
    p.write_bytes(_dump_bytes(8, 8, 80.0, px, px, px, px)[:-4])
    with pytest.raises(ValueError, match="truncated"):
        replay.read_positions(str(p))
    p.write_bytes(struct.pack("<ii4fi", -1, 8, 0, 0, 1, 1, 0))
    with pytest.raises(ValueError):
        replay.read_positions(str(p))
    d = tmp_path / "dens.bin"
    np.zeros(10, np.float32).tofile(d)
    with pytest.raises(ValueError):
        replay.read_density(str(d), 4, 4)


def test_empty_dump_round_trip(tmp_path):
    e = np.zeros(0, np.float32)
    d = replay.PositionDump(8, 8, 0.0, 0.0, 80.0, 80.0, e, e, e, e)
    p = tmp_path / "empty.bin"
    replay.write_positions(str(p), d)
    assert replay.read_positions(str(p)).nc == 0
