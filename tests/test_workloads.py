"""Seeded synthetic workloads: deterministic, inside the die, and of the
distributions the five configurations name."""
import numpy as np
import pytest


def test_generators_are_deterministic():
    from dpep import workloads
    a = workloads.small(3, seed=5, cells=5000, grid=64)
    b = workloads.small(3, seed=5, cells=5000, grid=64)
    c = workloads.small(3, seed=6, cells=5000, grid=64)
    for k in ("px", "py", "sx", "sy"):
        np.testing.assert_array_equal(getattr(a, k), getattr(b, k))
    assert not np.array_equal(a.px, c.px)
    np.testing.assert_array_equal(a.d0n, b.d0n)


@pytest.mark.parametrize("cfg", [1, 2, 3, 4, 5])
def test_cells_inside_die_and_sizes(cfg):
    from dpep import workloads
    w = workloads.small(cfg, seed=0, cells=20000, grid=64)
    assert w.px.dtype == np.float32
    assert (w.px >= w.xl).all() and (w.px + w.sx <= w.xh + 1e-3).all()
    assert (w.py >= w.yl).all() and (w.py + w.sy <= w.yh + 1e-3).all()
    assert set(np.unique(w.sy)) == {12.0}
    assert (w.sx >= 4).all() and (w.sx <= 200).all()
    mov = w.sx[: w.meta["movable"]]
    assert np.all(mov == np.round(mov))        # fillers are area / 12 wide
    assert w.d0n.shape == (w.M, w.N) and (w.d0n >= 0).all()


def test_width_distribution():
    from dpep import workloads
    rng = np.random.default_rng(0)
    wd = workloads.std_cell_widths(rng, 200000)
    assert wd.mean() == pytest.approx(8.2, abs=0.1)
    assert np.median(wd) == 7.0


def test_fixed_density_is_exact_macro_area():
    from dpep import workloads
    d = workloads.fixed_density([10.0], [20.0], [37.5], [11.0], 16, 16, 0, 0, 160, 160)
    assert d.sum() * 100.0 == pytest.approx(37.5 * 11.0)


def test_c5_displacement_is_seeded_and_clipped():
    from dpep import workloads
    w = workloads.small(5, cells=1000, grid=64)
    a = workloads.c5_displace(w, w.px, w.py, 3)
    b = workloads.c5_displace(w, w.px, w.py, 3)
    np.testing.assert_array_equal(a[0], b[0])
    assert (a[0] >= w.xl).all() and (a[0] + w.sx <= w.xh + 1e-3).all()


def test_headline_shape():
    from dpep import workloads
    w = workloads.config3()
    assert w.nc == 1_100_000 and (w.M, w.N) == (2048, 2048) and w.xh == 27000.0
