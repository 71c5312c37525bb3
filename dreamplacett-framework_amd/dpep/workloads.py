"""Seeded synthetic placements for the five electric-potential benchmark
configurations (random data of the shapes the benchmarks name; no netlists).

Every generator draws each array from its own sub-stream of
numpy.random.SeedSequence(seed), so arrays do not depend on each other's
draws.  Choices the configuration text leaves open are resolved here and
recorded in Workload.meta:

  * standard cells: height 12, width round(clip(lognormal(1.9, 0.6), 4, 200)),
    lower-left positions kept inside the die;
  * macros: sides uniform in the stated range, positions uniform inside the
    die, overlaps allowed; they enter only through the fixed-cell density D0;
  * D0n = target_density * (exact macro overlap area) / bin_area, the
    client-side initial_density_map / bin_area of the reference
    (integration/scatter_ttnn_client.py:786-795);
  * fillers fill max(0, die area - macro union - movable area) at the mean
    standard-cell area (width area/12, height 12) -- zero for the 210k design,
    whose macros cover the die;
  * C3 cluster centres: uniform in the middle 80 % of the die;
  * C4 macros: sides uniform in [300, 4000];
  * C5: die 27000, no macros, cells uniform in the centred 5 %-area square,
    per-step displacement N(0, 0.5 * bin) seeded by the step index.
"""
from __future__ import annotations

import dataclasses
from typing import Dict, Optional

import numpy as np

ROW_HEIGHT = 12.0


@dataclasses.dataclass
class Workload:
    name: str
    M: int
    N: int
    xl: float
    yl: float
    xh: float
    yh: float
    px: np.ndarray
    py: np.ndarray
    sx: np.ndarray
    sy: np.ndarray
    d0n: np.ndarray               # (M, N) float64
    meta: Dict[str, object]

    @property
    def nc(self) -> int:
        return int(self.px.size)

    @property
    def bsx(self) -> float:
        return (self.xh - self.xl) / self.M

    @property
    def bsy(self) -> float:
        return (self.yh - self.yl) / self.N

    def cells(self, dtype=np.float32):
        return tuple(np.ascontiguousarray(a, dtype=dtype)
                     for a in (self.px, self.py, self.sx, self.sy))


def _streams(seed: int, n: int):
    return [np.random.default_rng(s) for s in np.random.SeedSequence(seed).spawn(n)]


def std_cell_widths(rng: np.random.Generator, n: int) -> np.ndarray:
    w = rng.lognormal(mean=1.9, sigma=0.6, size=n)
    return np.round(np.clip(w, 4.0, 200.0))


def fixed_density(mx, my, mw, mh, M, N, xl, yl, xh, yh,
                  target_density: float = 1.0) -> np.ndarray:
    """Exact macro-overlap density per bin (float64, M x N), / bin area."""
    bsx, bsy = (xh - xl) / M, (yh - yl) / N
    d = np.zeros((M, N), dtype=np.float64)
    for x, y, w, h in zip(mx, my, mw, mh):
        kx0 = max(0, int(np.floor((x - xl) / bsx)))
        kx1 = min(M - 1, int(np.floor((x + w - xl) / bsx)))
        ky0 = max(0, int(np.floor((y - yl) / bsy)))
        ky1 = min(N - 1, int(np.floor((y + h - yl) / bsy)))
        if kx0 > kx1 or ky0 > ky1:
            continue
        kx = np.arange(kx0, kx1 + 1)
        ky = np.arange(ky0, ky1 + 1)
        tx = np.minimum(x + w, xl + (kx + 1) * bsx) - np.maximum(x, xl + kx * bsx)
        ty = np.minimum(y + h, yl + (ky + 1) * bsy) - np.maximum(y, yl + ky * bsy)
        d[kx0:kx1 + 1, ky0:ky1 + 1] += np.outer(np.maximum(tx, 0), np.maximum(ty, 0))
    return d * (target_density / (bsx * bsy))


def _macros(rng: np.random.Generator, count: int, lo: float, hi: float,
            die: float):
    w = rng.uniform(lo, hi, count)
    h = rng.uniform(lo, hi, count)
    x = rng.uniform(0.0, 1.0, count) * np.maximum(die - w, 0.0)
    y = rng.uniform(0.0, 1.0, count) * np.maximum(die - h, 0.0)
    return x, y, w, h


def _uniform_pos(rng, n, w, h, die):
    x = rng.uniform(0.0, 1.0, n) * (die - w)
    y = rng.uniform(0.0, 1.0, n) * (die - h)
    return x, y


def _gauss_pos(rng, n, cx, cy, sigma, w, h, die):
    x = rng.normal(0.0, sigma, n) + cx - 0.5 * w
    y = rng.normal(0.0, sigma, n) + cy - 0.5 * h
    return np.clip(x, 0.0, die - w), np.clip(y, 0.0, die - h)


def _finish(name, M, N, die, px, py, sx, sy, d0n, meta) -> Workload:
    f32 = np.float32
    return Workload(name=name, M=M, N=N, xl=0.0, yl=0.0, xh=float(die),
                    yh=float(die), px=px.astype(f32), py=py.astype(f32),
                    sx=sx.astype(f32), sy=sy.astype(f32), d0n=d0n, meta=meta)


def _design_210k(seed: int, n_mov: int, M: int, N: int, die: float):
    s = _streams(seed, 8)
    sx = std_cell_widths(s[0], n_mov)
    sy = np.full(n_mov, ROW_HEIGHT)
    mx, my, mw, mh = _macros(s[1], 540, 200.0, 1500.0, die)
    d0n = fixed_density(mx, my, mw, mh, M, N, 0.0, 0.0, die, die)
    ba = (die / M) * (die / N)
    union = float(np.minimum(d0n, 1.0).sum() * ba)
    mean_area = 98.5
    white = die * die - union - float((sx * sy).sum())
    n_fill = max(0, int(np.floor(white / mean_area)))
    fw = mean_area / ROW_HEIGHT
    sx = np.concatenate([sx, np.full(n_fill, fw)])
    sy = np.concatenate([sy, np.full(n_fill, ROW_HEIGHT)])
    meta = {"movable": n_mov, "fillers": n_fill, "macros": 540,
            "macro_union_area": union, "macro_sum_area": float((mw * mh).sum()),
            "die": die, "fixed_cells": (mx, my, mw, mh)}
    return s, sx, sy, d0n, meta


def config1(seed: int = 0, n_mov: int = 210_000, M: int = 512,
            N: int = 512) -> Workload:
    """210k cells + 540 macros, die 11600, 512x512, uniform positions."""
    die = 11600.0
    s, sx, sy, d0n, meta = _design_210k(seed, n_mov, M, N, die)
    px, py = _uniform_pos(s[2], sx.size, sx, sy, die)
    return _finish("C1", M, N, die, px, py, sx, sy, d0n, meta)


def config2(seed: int = 0, n_mov: int = 210_000, M: int = 2048,
            N: int = 2048) -> Workload:
    """C1's design at 2048x2048; 90 % Gaussian at the centre (die/8)."""
    die = 11600.0
    s, sx, sy, d0n, meta = _design_210k(seed, n_mov, M, N, die)
    n = sx.size
    n_g = int(round(0.9 * n))
    pick = s[3].permutation(n)
    g_idx, u_idx = pick[:n_g], pick[n_g:]
    px = np.empty(n)
    py = np.empty(n)
    px[g_idx], py[g_idx] = _gauss_pos(s[4], n_g, die / 2, die / 2, die / 8,
                                      sx[g_idx], sy[g_idx], die)
    px[u_idx], py[u_idx] = _uniform_pos(s[5], n - n_g, sx[u_idx], sy[u_idx], die)
    meta["gaussian_fraction"] = 0.9
    return _finish("C2", M, N, die, px, py, sx, sy, d0n, meta)


def config3(seed: int = 0, n_mov: int = 1_100_000, M: int = 2048,
            N: int = 2048, n_macros: int = 1300) -> Workload:
    """Headline: 1.1M cells, 1300 macros [300,4000], die 27000, 2048x2048,
    80 % uniform + 20 % in 4 Gaussian clusters (sigma die/20)."""
    die = 27000.0
    s = _streams(seed, 8)
    sx = std_cell_widths(s[0], n_mov)
    sy = np.full(n_mov, ROW_HEIGHT)
    mx, my, mw, mh = _macros(s[1], n_macros, 300.0, 4000.0, die)
    d0n = fixed_density(mx, my, mw, mh, M, N, 0.0, 0.0, die, die)
    centres = s[2].uniform(0.1 * die, 0.9 * die, size=(4, 2))
    pick = s[3].permutation(n_mov)
    n_c = int(round(0.2 * n_mov))
    c_idx, u_idx = pick[:n_c], pick[n_c:]
    px = np.empty(n_mov)
    py = np.empty(n_mov)
    px[u_idx], py[u_idx] = _uniform_pos(s[4], u_idx.size, sx[u_idx], sy[u_idx], die)
    which = s[5].integers(0, 4, n_c)
    gx = s[6].normal(0.0, die / 20, n_c)
    gy = s[7].normal(0.0, die / 20, n_c)
    w, h = sx[c_idx], sy[c_idx]
    px[c_idx] = np.clip(centres[which, 0] + gx - 0.5 * w, 0.0, die - w)
    py[c_idx] = np.clip(centres[which, 1] + gy - 0.5 * h, 0.0, die - h)
    ba = (die / M) * (die / N)
    meta = {"movable": n_mov, "macros": n_macros, "die": die,
            "fixed_cells": (mx, my, mw, mh),
            "cluster_centres": centres.tolist(), "cluster_fraction": 0.2,
            "macro_union_area_fraction": float(np.minimum(d0n, 1.0).sum() * ba / die ** 2)}
    return _finish("C3", M, N, die, px, py, sx, sy, d0n, meta)


def config4(seed: int = 0, n_mov: int = 2_000_000, M: int = 4096,
            N: int = 4096, n_macros: int = 2000) -> Workload:
    """2.0M cells, 2000 macros [300,4000], die 36000, 4096x4096, uniform."""
    die = 36000.0
    s = _streams(seed, 8)
    sx = std_cell_widths(s[0], n_mov)
    sy = np.full(n_mov, ROW_HEIGHT)
    mx, my, mw, mh = _macros(s[1], n_macros, 300.0, 4000.0, die)
    d0n = fixed_density(mx, my, mw, mh, M, N, 0.0, 0.0, die, die)
    px, py = _uniform_pos(s[2], n_mov, sx, sy, die)
    meta = {"movable": n_mov, "macros": n_macros, "die": die,
            "fixed_cells": (mx, my, mw, mh)}
    return _finish("C4", M, N, die, px, py, sx, sy, d0n, meta)


def config5(seed: int = 0, n_mov: int = 1_100_000, M: int = 512,
            N: int = 512) -> Workload:
    """1.1M cells in the centred 5 %-area square of a 27000 die, 512x512."""
    die = 27000.0
    s = _streams(seed, 4)
    sx = std_cell_widths(s[0], n_mov)
    sy = np.full(n_mov, ROW_HEIGHT)
    side = die * np.sqrt(0.05)
    lo = 0.5 * (die - side)
    px = lo + s[1].uniform(0.0, 1.0, n_mov) * (side - sx)
    py = lo + s[2].uniform(0.0, 1.0, n_mov) * (side - sy)
    d0n = np.zeros((M, N))
    meta = {"movable": n_mov, "macros": 0, "die": die, "square_side": side}
    return _finish("C5", M, N, die, px, py, sx, sy, d0n, meta)


def c5_displace(w: Workload, px: np.ndarray, py: np.ndarray, step: int):
    """Step `step`'s positions: + N(0, 0.5 bin) per cell (seed = step),
    clipped to the die; returns float32 arrays."""
    rng = np.random.default_rng(step)
    dx = rng.normal(0.0, 0.5 * w.bsx, px.size)
    dy = rng.normal(0.0, 0.5 * w.bsy, py.size)
    nx = np.clip(px.astype(np.float64) + dx, w.xl, w.xh - w.sx)
    ny = np.clip(py.astype(np.float64) + dy, w.yl, w.yh - w.sy)
    return nx.astype(np.float32), ny.astype(np.float32)


def walk(w: Workload, steps: int, first: int = 0):
    """Positions of `steps` consecutive steps of the seeded drift: step k's
    positions are step k-1's (the placement's, for the first) plus
    c5_displace with seed first + k.  Yields (step, px, py), float32.  The
    100-step loop of the extreme-hotspot configuration is walk(config5(),
    100); the same drift applied to another placement gives it cells that
    move a fraction of a bin per step, as early placement iterations do."""
    px, py = w.px, w.py
    for k in range(steps):
        px, py = c5_displace(w, px, py, first + k)
        yield first + k, px, py


CONFIGS = {1: config1, 2: config2, 3: config3, 4: config4, 5: config5}


def make(cfg: int, seed: int = 0, **kw) -> Workload:
    return CONFIGS[int(cfg)](seed=seed, **kw)


def small(cfg: int, seed: int = 0, cells: Optional[int] = None,
          grid: Optional[int] = None) -> Workload:
    """A scaled-down instance of a configuration (same recipe, fewer cells,
    smaller grid) for quick parity checks."""
    kw = {}
    if cells is not None:
        kw["n_mov"] = cells
    if grid is not None:
        kw["M"] = kw["N"] = grid
    if cfg in (3, 4) and cells is not None:
        kw["n_macros"] = max(4, cells // 1000)
    return make(cfg, seed, **kw)
