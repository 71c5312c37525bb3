"""Filler cells for the electric-potential step, sized and seeded the way
DREAMPlace's PlaceDB does it.

The reference repository receives fillers ready-made: they are the tail of
DREAMPlace's position vector, ``[movable | fixed terminals | filler]``
(integration/scatter_ttnn_client.py:611-617), and their sizes come with the
other node sizes.  DREAMPlace itself is not vendored, so the rules below are
its published behaviour as recalled, not checked against its source (the
sizing is "parity unpinned"):

  * width  = mean width of the movable cells ranked between the 5th and the
             95th percentile of the width order (the 5 % narrowest and widest
             cells are left out); 0 when that range is empty;
  * height = the row height;
  * placeable area = max(die area - fixed area inside the die,
                         total space area of the rows, when given);
  * filler area    = max(0, target_density * placeable area - movable area);
  * count          = round(filler area / (width * height));
  * initial positions: lower-left corners uniform in
                       [xl, xh - width] x [yl, yh - height].

The fixed area is the sum over fixed cells of their area clipped to the die
(overlapping macros count twice, as a sum of node areas does).
"""
from __future__ import annotations

import dataclasses
from typing import Optional, Tuple

import numpy as np


@dataclasses.dataclass
class Fillers:
    n: int
    width: float
    height: float
    px: np.ndarray          # lower-left x, n values
    py: np.ndarray          # lower-left y, n values

    def sizes(self, dtype=np.float64) -> Tuple[np.ndarray, np.ndarray]:
        return (np.full(self.n, self.width, dtype), np.full(self.n, self.height, dtype))


def filler_width(movable_sx: np.ndarray) -> float:
    """Mean width of the movable cells between the 5th and 95th percentile
    of the width order."""
    w = np.asarray(movable_sx, dtype=np.float64)
    n = w.size
    lo, hi = int(n * 0.05), int(n * 0.95)
    if lo >= hi:
        return 0.0
    order = np.argsort(w, kind="stable")
    return float(np.mean(w[order[lo:hi]]))


def fixed_area_in_die(px, py, sx, sy, xl: float, yl: float, xh: float, yh: float) -> float:
    """Sum of the fixed cells' areas clipped to the die."""
    px, py, sx, sy = (np.asarray(a, dtype=np.float64) for a in (px, py, sx, sy))
    wx = np.maximum(np.minimum(px + sx, xh) - np.maximum(px, xl), 0.0)
    wy = np.maximum(np.minimum(py + sy, yh) - np.maximum(py, yl), 0.0)
    return float(np.sum(wx * wy))


def filler_count(width: float, height: float, movable_area: float, fixed_area: float,
                 die_area: float, target_density: float,
                 total_space_area: Optional[float] = None) -> int:
    """round(max(0, target_density * placeable - movable) / (width * height))."""
    if not (target_density >= 0.0):
        raise ValueError(f"target_density={target_density} must be >= 0")
    if width <= 0.0 or height <= 0.0:
        return 0
    placeable = die_area - fixed_area
    if total_space_area is not None:
        placeable = max(placeable, float(total_space_area))
    area = max(placeable * target_density - movable_area, 0.0)
    return int(round(area / (width * height)))


def make_fillers(movable_sx, movable_sy, row_height: float, xl: float, yl: float,
                 xh: float, yh: float, target_density: float, fixed_area: float = 0.0,
                 total_space_area: Optional[float] = None, seed: int = 0) -> Fillers:
    """Sizes, count and seeded initial positions of the filler cells."""
    if not (xh > xl and yh > yl):
        raise ValueError("empty die")
    msx = np.asarray(movable_sx, dtype=np.float64)
    msy = np.asarray(movable_sy, dtype=np.float64)
    if msx.shape != msy.shape:
        raise ValueError("movable_sx and movable_sy differ in length")
    w, h = filler_width(msx), float(row_height)
    n = filler_count(w, h, float(np.sum(msx * msy)), float(fixed_area),
                     (xh - xl) * (yh - yl), target_density, total_space_area)
    rng = np.random.default_rng(seed)
    px = rng.uniform(xl, max(xl, xh - w), n)
    py = rng.uniform(yl, max(yl, yh - h), n)
    return Fillers(n, w, h, px, py)
