"""Shared-memory wire format between the electric-potential client and the
server process (integration/scatter_ttnn_client.py:151-163, :224-271 and
host/density_scatter_ttnn_server_host.cpp:37-53, :1269-1290 of the
reference).

File ``<ipc_dir>/scatter.shm``, little endian, created and sized by the
client, mapped MAP_SHARED by both sides.

Version 1 (the reference layout, unchanged):
    header, 64 bytes
        [0:4]   state        u32  0 idle, 1 go, 2 done, 3 quit
        [4:8]   nc_actual    i32
        [8:44]  timing[9]    f32  h2d scatter gather d2h_den upload compute
                                  download fw total (milliseconds)
        [44:48] gather_mode  u32
        [48:64] padding
    px, py, sx, sy           f32 [soa_padded] each, soa_padded =
                             ceil(nc_max / 1024) * 1024
    field_x, field_y         f32 [M*N] each
    init_density             f32 [M*N] (initial_density_map / bin_area,
                             written once by the client)

Version 2 = version 1 plus, after init_density:
    density, potential       f32 [M*N] each
    grad_x, grad_y           f32 [soa_padded] each (per-cell field gather)
and, in the header padding:
        [48:52] magic        u32  0x32504544 ("DEP2")
        [52:56] version      u32  2
        [56:60] outputs      u32  bit 0 density, bit 1 potential, bit 2 grads,
                                  bit 3 no fields (field_x/field_y not written),
                                  bit 4 keep sizes (sx/sy not rewritten for
                                  this step: the server keeps the sizes of
                                  its last step with at least nc cells)
A version-1 server ignores bytes 48..64; a version-1 client never writes the
magic, so the server falls back to the version-1 layout.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass

STATE_IDLE = 0
STATE_GO = 1
STATE_DONE = 2
STATE_QUIT = 3

HEADER_SIZE = 64
OFF_STATE = 0
OFF_NC = 4
OFF_TIMINGS = 8
OFF_GMODE = 44
OFF_MAGIC = 48
OFF_VERSION = 52
OFF_OUTPUTS = 56

MAGIC_V2 = 0x32504544
OUT_DENSITY = 0x1
OUT_POTENTIAL = 0x2
OUT_GRADS = 0x4
OUT_NO_FIELDS = 0x8
IN_KEEP_SIZES = 0x10

# state nc h2d scatter gather d2h_den upload compute download fw total gm
HDR_TIMING_FMT = "<IifffffffffI"
TIMING_KEYS = ("h2d_ms", "scatter_ms", "gather_ms", "d2h_density_ms",
               "ttnn_upload_ms", "ttnn_compute_ms", "ttnn_download_ms",
               "fw_ms", "total_server_ms")

# gather_mode values the reference client knows, plus this server's own.
GATHER_MODE_HIP = 16
GATHER_MODE_NAMES = {0: "v6", 1: "v7", 2: "v8", 3: "v9", 4: "v10", 5: "v11",
                     GATHER_MODE_HIP: "hip"}


def soa_padded(nc_max: int) -> int:
    return ((int(nc_max) + 1023) // 1024) * 1024


@dataclass(frozen=True)
class Layout:
    """Byte offsets of every slot for one (M, N, nc_max, version)."""
    M: int
    N: int
    nc_max: int
    version: int = 2

    @property
    def soa(self) -> int:
        return soa_padded(self.nc_max)

    @property
    def pos_bytes(self) -> int:
        return self.soa * 4

    @property
    def map_bytes(self) -> int:
        return self.M * self.N * 4

    def offset(self, name: str) -> int:
        o = HEADER_SIZE
        order = ["px", "py", "sx", "sy", "field_x", "field_y", "init_density"]
        if self.version >= 2:
            order += ["density", "potential", "grad_x", "grad_y"]
        sizes = {"px": self.pos_bytes, "py": self.pos_bytes,
                 "sx": self.pos_bytes, "sy": self.pos_bytes,
                 "grad_x": self.pos_bytes, "grad_y": self.pos_bytes}
        for n in order:
            if n == name:
                return o
            o += sizes.get(n, self.map_bytes)
        raise KeyError(f"slot {name!r} not in version {self.version} layout")

    @property
    def total_size(self) -> int:
        base = HEADER_SIZE + 4 * self.pos_bytes + 3 * self.map_bytes
        if self.version >= 2:
            base += 2 * self.map_bytes + 2 * self.pos_bytes
        return base


def write_v2_header(buf, outputs: int = OUT_DENSITY | OUT_POTENTIAL | OUT_GRADS) -> None:
    struct.pack_into("<III", buf, OFF_MAGIC, MAGIC_V2, 2, outputs)


def set_outputs(buf, outputs: int) -> None:
    """The outputs word a version-2 server reads before every step."""
    struct.pack_into("<I", buf, OFF_OUTPUTS, outputs)


def outputs_of(names) -> int:
    """Outputs word for a set of output names (density, potential, field_x,
    field_y, grad_x, grad_y)."""
    names = set(names)
    word = 0 if names & {"field_x", "field_y"} else OUT_NO_FIELDS
    if "density" in names:
        word |= OUT_DENSITY
    if "potential" in names:
        word |= OUT_POTENTIAL
    if names & {"grad_x", "grad_y"}:
        word |= OUT_GRADS
    return word


def read_timings(buf):
    vals = struct.unpack_from(HDR_TIMING_FMT, buf, 0)
    timings = dict(zip(TIMING_KEYS, (float(v) for v in vals[2:11])))
    return vals[0], vals[1], timings, int(vals[11])
