"""Pins the float64 oracle (oracle/dpep_oracle.c) before anything is compared
with it: golden vectors written by scipy.fft and by plain Python loops
(tests/golden/), brute force on tiny inputs, invariants and closed forms.
Each check is chosen so that a plausible slip in the oracle (a dropped term, a
wrong sign or index, a transposed operand, a missing stretch) fails it.
"""
import os

import numpy as np
import pytest

from conftest import rel_l2, rel_linf

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def spectral_golden():
    return np.load(os.path.join(GOLDEN, "spectral_golden.npz"))


@pytest.fixture(scope="module")
def density_golden():
    return np.load(os.path.join(GOLDEN, "density_golden.npz"))


# --------------------------------------------------------------------------
# 1-D transforms against scipy.fft golden vectors
# --------------------------------------------------------------------------
@pytest.mark.parametrize("K", [8, 12, 16, 64])
@pytest.mark.parametrize("kind,key", [(0, "dct2"), (1, "idct"), (2, "idxst")])
def test_line_transform_matches_scipy(oracle, spectral_golden, K, kind, key):
    x = spectral_golden[f"x_{K}"]
    got = oracle.line_transform(kind, x)
    np.testing.assert_allclose(got, spectral_golden[f"{key}_{K}"], rtol=0, atol=1e-12)


# --------------------------------------------------------------------------
# 2-D solve: FFT path and direct-matrix path against scipy golden vectors
# --------------------------------------------------------------------------
@pytest.mark.parametrize("tag", ["8x8", "16x8", "8x32"])
@pytest.mark.parametrize("direct", [False, True])
def test_solve_matches_scipy(oracle, spectral_golden, tag, direct):
    rho = spectral_golden[f"rho_{tag}"]
    bsx, bsy = spectral_golden[f"geom_{tag}"]
    phi, fx, fy = oracle.solve(rho, bsx, bsy, direct=direct)
    for name, got in (("fx", fx), ("fy", fy), ("phi", phi)):
        want = spectral_golden[f"{name}_{tag}"]
        assert rel_linf(got, want) < 1e-12, name


@pytest.mark.parametrize("M,N", [(16, 16), (32, 8), (8, 64), (24, 20)])
def test_solve_fft_equals_direct_matrices(oracle, M, N):
    rng = np.random.default_rng(M * 100 + N)
    rho = rng.random((M, N))
    a = oracle.solve(rho, 2.5, 1.5, direct=False)
    b = oracle.solve(rho, 2.5, 1.5, direct=True)
    for x, y in zip(a, b):
        assert rel_linf(x, y) < 1e-11


@pytest.mark.parametrize("u0,v0", [(3, 2), (1, 0), (0, 5), (7, 7)])
def test_single_mode_closed_form(oracle, u0, v0):
    """rho = cos(pi u0 (x+1/2)/M) cos(pi v0 (y+1/2)/N): A has one nonzero
    (value c_u c_v / 4 with c_0 = 2, c_k>0 = 1) and phi, fx, fy are single
    products with amplitudes fixed by w_u, w_v (fields = -bsx grad phi)."""
    M, N, bsx, bsy = 16, 32, 3.0, 2.0
    t = (np.arange(M)[:, None] + 0.5)
    s = (np.arange(N)[None, :] + 0.5)
    rho = np.cos(np.pi * u0 * t / M) * np.cos(np.pi * v0 * s / N)
    phi, fx, fy = oracle.solve(rho, bsx, bsy)
    wu = 2 * np.pi * u0 / M
    wv = 2 * np.pi * v0 / N * bsx / bsy
    D = wu * wu + wv * wv
    amp = (2.0 if u0 == 0 else 1.0) * (2.0 if v0 == 0 else 1.0)   # A[u0,v0]
    cu = 1.0 if u0 == 0 else 2.0
    cv = 1.0 if v0 == 0 else 2.0
    want_phi = amp * cu * cv / D * rho
    want_fx = amp * cv * (wu / D) * np.sin(np.pi * u0 * t / M) * np.cos(np.pi * v0 * s / N)
    want_fy = amp * cu * (wv / D) * np.cos(np.pi * u0 * t / M) * np.sin(np.pi * v0 * s / N)
    np.testing.assert_allclose(phi, want_phi, atol=1e-10 * np.abs(want_phi).max())
    np.testing.assert_allclose(fx, want_fx, atol=1e-10 * max(np.abs(want_fx).max(), 1))
    np.testing.assert_allclose(fy, want_fy, atol=1e-10 * max(np.abs(want_fy).max(), 1))
    # Poisson: -(d2/dt2 + (bsx/bsy)^2 d2/ds2) phi = rho for a single mode
    lap = ((np.pi * u0 / M) ** 2 + (np.pi * v0 / N * bsx / bsy) ** 2)
    np.testing.assert_allclose(lap * phi, amp * cu * cv / 4 * rho, atol=1e-10)


def test_constant_density_gives_zero_field(oracle):
    rho = np.full((16, 16), 0.7)
    phi, fx, fy = oracle.solve(rho, 1.0, 1.0)
    assert np.abs(phi).max() < 1e-12 and np.abs(fx).max() < 1e-12 and np.abs(fy).max() < 1e-12


def test_field_is_minus_gradient_of_potential(oracle):
    """Smooth density: centred differences of phi match (fx, fy) = -bsx grad phi."""
    M = N = 128
    bsx, bsy = 2.0, 1.0
    x = (np.arange(M)[:, None] + 0.5) / M
    y = (np.arange(N)[None, :] + 0.5) / N
    rho = np.exp(-((x - 0.5) ** 2 + (y - 0.4) ** 2) / 0.02)
    phi, fx, fy = oracle.solve(rho, bsx, bsy)
    dphx = (phi[2:, :] - phi[:-2, :]) / 2.0                  # per x-bin
    dphy = (phi[:, 2:] - phi[:, :-2]) / 2.0 * (bsx / bsy)    # per y-bin, scaled
    assert rel_l2(-dphx[:, 8:-8], fx[1:-1, 8:-8]) < 5e-3
    assert rel_l2(-dphy[8:-8, :], fy[8:-8, 1:-1]) < 5e-3


# --------------------------------------------------------------------------
# Density scatter
# --------------------------------------------------------------------------
@pytest.mark.parametrize("stretch", [True, False])
def test_density_matches_loop_golden(oracle, density_golden, stretch):
    g = density_golden
    M, N = int(g["geom"][0]), int(g["geom"][1])
    xl, yl, xh, yh = map(float, g["geom"][2:])
    rho = oracle.density(g["px"], g["py"], g["sx"], g["sy"], M, N, xl, yl, xh, yh,
                         stretch=stretch)
    want = g["rho_stretch" if stretch else "rho_nostretch"]
    np.testing.assert_allclose(rho, want, rtol=0, atol=1e-12)


@pytest.mark.parametrize("stretch", [True, False])
def test_density_equals_bruteforce(oracle, stretch):
    rng = np.random.default_rng(3)
    M, N, xl, yl, xh, yh = 20, 24, 0.0, 0.0, 100.0, 60.0
    n = 300
    px = rng.uniform(-10, 105, n); py = rng.uniform(-10, 62, n)
    sx = rng.uniform(0.1, 14, n); sy = rng.uniform(0.1, 6, n)
    a = oracle.density(px, py, sx, sy, M, N, xl, yl, xh, yh, stretch)
    b = oracle.density(px, py, sx, sy, M, N, xl, yl, xh, yh, stretch, brute=True)
    np.testing.assert_allclose(a, b, rtol=0, atol=1e-12)


def test_mass_conservation_with_stretch(oracle):
    """Cells inside the die: sum(rho) * bin_area = sum(sx * sy) exactly, the
    stretch being area preserving through ratio."""
    rng = np.random.default_rng(4)
    M = N = 32
    die = 320.0
    n = 2000
    sx = rng.uniform(0.5, 30, n); sy = rng.uniform(0.5, 20, n)
    # keep stretched extents inside the die
    px = rng.uniform(20, die - 50, n); py = rng.uniform(20, die - 40, n)
    rho = oracle.density(px, py, sx, sy, M, N, 0, 0, die, die, True)
    ba = (die / M) * (die / N)
    assert rho.sum() * ba == pytest.approx((sx * sy).sum(), rel=1e-12)


def test_translation_by_whole_bins(oracle):
    rng = np.random.default_rng(5)
    M = N = 32
    die = 64.0
    n = 200
    px = rng.uniform(10, 30, n); py = rng.uniform(10, 30, n)
    sx = rng.uniform(0.2, 5, n); sy = rng.uniform(0.2, 5, n)
    a = oracle.density(px, py, sx, sy, M, N, 0, 0, die, die)
    b = oracle.density(px + 3 * 2.0, py + 5 * 2.0, sx, sy, M, N, 0, 0, die, die)
    np.testing.assert_allclose(b[3:, 5:], a[:-3, :-5], atol=1e-12)


def test_permutation_invariance_and_padding(oracle):
    rng = np.random.default_rng(6)
    n = 500
    px = rng.uniform(0, 90, n); py = rng.uniform(0, 90, n)
    sx = rng.uniform(0.5, 8, n); sy = rng.uniform(0.5, 8, n)
    a = oracle.density(px, py, sx, sy, 16, 16, 0, 0, 100, 100)
    p = rng.permutation(n)
    # zero-size, NaN and out-of-die padding cells contribute nothing
    pad = 5
    px2 = np.concatenate([px[p], [0, np.nan, 500, 1, -400]])
    py2 = np.concatenate([py[p], [0, 1, 500, np.inf, -400]])
    sx2 = np.concatenate([sx[p], [0, 1, 2, 3, 4]])
    sy2 = np.concatenate([sy[p], [0, 1, 2, 3, 4]])
    b = oracle.density(px2, py2, sx2, sy2, 16, 16, 0, 0, 100, 100)
    np.testing.assert_allclose(a, b, rtol=1e-13, atol=1e-13)
    assert pad == 5


def test_initial_density_is_added(oracle):
    rng = np.random.default_rng(8)
    d0 = rng.random((16, 16))
    px = rng.uniform(0, 90, 50); py = rng.uniform(0, 90, 50)
    s = np.full(50, 4.0)
    a = oracle.density(px, py, s, s, 16, 16, 0, 0, 100, 100)
    b = oracle.density(px, py, s, s, 16, 16, 0, 0, 100, 100, d0n=d0)
    np.testing.assert_allclose(b - a, d0, atol=1e-13)


# --------------------------------------------------------------------------
# Per-cell gather
# --------------------------------------------------------------------------
def test_gather_is_adjoint_of_scatter(oracle):
    """sum_i gx_i(f) = sum_b f[b] * rho_cells[b] * bin_area."""
    rng = np.random.default_rng(9)
    M, N, die = 24, 16, 96.0
    n = 400
    px = rng.uniform(-5, 95, n); py = rng.uniform(-5, 95, n)
    sx = rng.uniform(0.3, 10, n); sy = rng.uniform(0.3, 9, n)
    f = rng.standard_normal((M, N))
    rho = oracle.density(px, py, sx, sy, M, N, 0, 0, die, die)
    gx, gy = oracle.gather(px, py, sx, sy, M, N, 0, 0, die, die, f, -f)
    ba = (die / M) * (die / N)
    assert gx.sum() == pytest.approx((f * rho).sum() * ba, rel=1e-12)
    assert gy.sum() == pytest.approx(-(f * rho).sum() * ba, rel=1e-12)


def test_gather_constant_field_gives_cell_area(oracle):
    rng = np.random.default_rng(10)
    n = 300
    px = rng.uniform(20, 70, n); py = rng.uniform(20, 70, n)
    sx = rng.uniform(0.3, 10, n); sy = rng.uniform(0.3, 9, n)
    f = np.full((16, 16), 2.5)
    gx, gy = oracle.gather(px, py, sx, sy, 16, 16, 0, 0, 100, 100, f, f)
    np.testing.assert_allclose(gx, 2.5 * sx * sy, rtol=1e-12)
    np.testing.assert_allclose(gy, 2.5 * sx * sy, rtol=1e-12)


def test_gather_matches_bruteforce(oracle):
    rng = np.random.default_rng(11)
    M, N, die = 12, 10, 60.0
    n = 40
    px = rng.uniform(-3, 58, n); py = rng.uniform(-3, 58, n)
    sx = rng.uniform(0.3, 12, n); sy = rng.uniform(0.3, 12, n)
    f = rng.standard_normal((M, N))
    gx, _ = oracle.gather(px, py, sx, sy, M, N, 0, 0, die, die, f, f)
    bsx, bsy = die / M, die / N
    want = np.zeros(n)
    for i in range(n):
        w, h = max(sx[i], np.sqrt(2) * bsx), max(sy[i], np.sqrt(2) * bsy)
        x, y = px[i] + (sx[i] - w) / 2, py[i] + (sy[i] - h) / 2
        r = sx[i] * sy[i] / (w * h)
        for k in range(M):
            tx = max(0.0, min(x + w, (k + 1) * bsx) - max(x, k * bsx))
            for q in range(N):
                ty = max(0.0, min(y + h, (q + 1) * bsy) - max(y, q * bsy))
                want[i] += r * tx * ty * f[k, q]
    np.testing.assert_allclose(gx, want, rtol=1e-12, atol=1e-12)


def test_planted_mistakes_are_caught(oracle, spectral_golden):
    """The golden checks above would fail for typical slips: a missing factor
    2 in S_M, a flipped sign, swapped fields, transposed axes, a dropped
    stretch ratio."""
    rho = spectral_golden["rho_16x8"]
    bsx, bsy = spectral_golden["geom_16x8"]
    phi, fx, fy = oracle.solve(rho, bsx, bsy)
    assert rel_linf(fx / 2.0, spectral_golden["fx_16x8"]) > 0.1
    assert rel_linf(-fx, spectral_golden["fx_16x8"]) > 0.1
    assert rel_linf(fy, spectral_golden["fx_16x8"]) > 0.1
    phi_t, _, _ = oracle.solve(rho.T.copy(), bsy, bsx)
    assert rel_linf(phi_t.T, spectral_golden["phi_16x8"]) > 1e-3
    px = np.array([10.0]); py = np.array([10.0]); s = np.array([1.0])
    a = oracle.density(px, py, s, s, 8, 8, 0, 0, 80, 80, stretch=True)
    b = oracle.density(px, py, s, s, 8, 8, 0, 0, 80, 80, stretch=False)
    assert a.sum() == pytest.approx(b.sum())      # ratio keeps the mass ...
    assert not np.allclose(a, b)                  # ... but spreads it
