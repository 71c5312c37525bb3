"""Filler sizing and placement (dpep.fillers), checked against hand-computed
cases and the area balance the rules imply."""
import numpy as np
import pytest

from dpep import fillers


def test_width_drops_the_narrowest_and_widest_five_percent():
    w = np.arange(1.0, 101.0)                  # 100 cells, widths 1..100
    np.random.default_rng(0).shuffle(w)
    # ranks 5..94 of the width order are the widths 6..95
    assert fillers.filler_width(w) == pytest.approx(np.mean(np.arange(6.0, 96.0)))


def test_width_of_too_few_cells_is_zero():
    assert fillers.filler_width(np.array([3.0])) == 0.0
    assert fillers.filler_width(np.array([])) == 0.0


def test_fixed_area_is_clipped_to_the_die():
    # one macro half outside on x, one fully inside, one fully outside
    px = np.array([-5.0, 20.0, 200.0]); py = np.array([0.0, 20.0, 0.0])
    sx = np.array([10.0, 4.0, 10.0]); sy = np.array([10.0, 5.0, 10.0])
    assert fillers.fixed_area_in_die(px, py, sx, sy, 0, 0, 100, 100) == pytest.approx(50 + 20)


def test_count_hand_case():
    # die 100 x 100, fixed 1000, movable 3000, target 0.9:
    # 0.9 * 9000 - 3000 = 5100 -> 5100 / (5 * 12) = 85
    assert fillers.filler_count(5.0, 12.0, 3000.0, 1000.0, 10000.0, 0.9) == 85
    # the rows' space area wins when larger than die - fixed
    assert fillers.filler_count(5.0, 12.0, 3000.0, 1000.0, 10000.0, 0.9,
                                total_space_area=9500.0) == round((0.9 * 9500 - 3000) / 60)
    # movable area above the target: no fillers
    assert fillers.filler_count(5.0, 12.0, 9000.0, 1000.0, 10000.0, 0.9) == 0
    with pytest.raises(ValueError):
        fillers.filler_count(5.0, 12.0, 0.0, 0.0, 1.0, -1.0)


def test_area_balance_positions_and_seed():
    rng = np.random.default_rng(3)
    sx = np.round(np.clip(rng.lognormal(1.9, 0.6, 5000), 4, 200))
    sy = np.full(sx.size, 12.0)
    f = fillers.make_fillers(sx, sy, 12.0, 0.0, 0.0, 2000.0, 1500.0, 0.8,
                             fixed_area=2.5e5, seed=7)
    target = 0.8 * (2000.0 * 1500.0 - 2.5e5) - float(np.sum(sx * sy))
    # the count rounds: total filler area within half a filler of the target
    assert abs(f.n * f.width * f.height - target) <= 0.5 * f.width * f.height + 1e-6
    assert f.height == 12.0 and f.px.size == f.n == f.py.size
    assert np.all(f.px >= 0.0) and np.all(f.px + f.width <= 2000.0)
    assert np.all(f.py >= 0.0) and np.all(f.py + f.height <= 1500.0)
    g = fillers.make_fillers(sx, sy, 12.0, 0.0, 0.0, 2000.0, 1500.0, 0.8,
                             fixed_area=2.5e5, seed=7)
    assert np.array_equal(f.px, g.px) and np.array_equal(f.py, g.py)
    fsx, fsy = f.sizes(np.float32)
    assert fsx.dtype == np.float32 and np.all(fsx == np.float32(f.width))
