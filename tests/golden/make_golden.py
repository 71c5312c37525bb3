"""Writes tests/golden/*.npz: golden vectors that pin the oracle independently
of its own code.

spectral_golden.npz -- 1-D and 2-D transforms computed with scipy.fft (DCT-II,
  DCT-III, DST-III), mapped onto the reference's matrix conventions
  (host/density_scatter_ttnn_server_host.cpp:124-181):
     C_K x  = dct(x, type=2) / K
     I_K X  = dct(X, type=3)                    (X[0] + 2 sum_k X[k] cos ...)
     S_K X  = dst([X[1:], 0], type=3) / 2       (sum_k X[k] sin(pi k (n+1/2)/K))
  and the 2-D step A = C_M rho C_N^T, fx = 2 S_M (A.Wx) I_N^T,
  fy = 2 I_M (A.Wy) S_N^T, phi = I_M (A/D) I_N^T on small grids.
density_golden.npz -- tiny placements whose density is written with plain
  Python loops over every (cell, bin) pair in float64 (no span logic).

Run: python tests/golden/make_golden.py   (needs scipy; only in this
container -- the fixtures, not scipy, travel with the tests).
"""
import os

import numpy as np
import scipy.fft as sf

HERE = os.path.dirname(os.path.abspath(__file__))


def c_k(x):
    return sf.dct(x, type=2, axis=-1) / x.shape[-1]


def i_k(X):
    return sf.dct(X, type=3, axis=-1)


def s_k(X):
    Xs = np.concatenate([X[..., 1:], np.zeros_like(X[..., :1])], axis=-1)
    return sf.dst(Xs, type=3, axis=-1) / 2.0


def along(f, a, axis):
    return np.moveaxis(f(np.moveaxis(a, axis, -1)), -1, axis)


def weights(M, N, bsx, bsy):
    wu = 2 * np.pi * np.arange(M)[:, None] / M
    wv = 2 * np.pi * np.arange(N)[None, :] / N * (bsx / bsy)
    D = wu ** 2 + wv ** 2
    D[0, 0] = 1.0
    Wx, Wy, iD = wu / (2 * D), wv / (2 * D), 1.0 / D
    Wx[0, 0] = Wy[0, 0] = iD[0, 0] = 0.0
    return Wx, Wy, iD


def spectral():
    rng = np.random.default_rng(20251201)
    out = {}
    for K in (8, 12, 16, 64):
        x = rng.standard_normal(K)
        out[f"x_{K}"] = x
        out[f"dct2_{K}"] = c_k(x) * K / 2.0         # unscaled sum x cos
        out[f"idct_{K}"] = i_k(x)
        out[f"idxst_{K}"] = s_k(x)
    for (M, N, bsx, bsy) in ((8, 8, 1.0, 1.0), (16, 8, 3.0, 2.0), (8, 32, 1.5, 4.0)):
        rho = rng.random((M, N))
        A = along(c_k, along(c_k, rho, 0), 1)
        Wx, Wy, iD = weights(M, N, bsx, bsy)
        fx = 2.0 * along(s_k, along(i_k, A * Wx, 1), 0)
        fy = 2.0 * along(i_k, along(s_k, A * Wy, 1), 0)
        phi = along(i_k, along(i_k, A * iD, 1), 0)
        tag = f"{M}x{N}"
        out[f"rho_{tag}"] = rho
        out[f"geom_{tag}"] = np.array([bsx, bsy])
        out[f"fx_{tag}"] = fx
        out[f"fy_{tag}"] = fy
        out[f"phi_{tag}"] = phi
    np.savez_compressed(os.path.join(HERE, "spectral_golden.npz"), **out)


def loop_density(px, py, sx, sy, M, N, xl, yl, xh, yh, stretch):
    bsx, bsy = (xh - xl) / M, (yh - yl) / N
    rho = np.zeros((M, N))
    for i in range(len(px)):
        if not (sx[i] > 0 and sy[i] > 0):
            continue
        w, h, x, y, r = sx[i], sy[i], px[i], py[i], 1.0
        if stretch:
            w, h = max(sx[i], np.sqrt(2) * bsx), max(sy[i], np.sqrt(2) * bsy)
            x, y = px[i] + (sx[i] - w) / 2, py[i] + (sy[i] - h) / 2
            r = sx[i] * sy[i] / (w * h)
        for k in range(M):
            tx = max(0.0, min(x + w, xl + (k + 1) * bsx) - max(x, xl + k * bsx))
            for q in range(N):
                ty = max(0.0, min(y + h, yl + (q + 1) * bsy) - max(y, yl + q * bsy))
                rho[k, q] += r * tx * ty / (bsx * bsy)
    return rho


def density():
    rng = np.random.default_rng(7)
    out = {}
    M, N, xl, yl, xh, yh = 12, 10, -3.0, 2.0, 45.0, 32.0
    n = 60
    bsx, bsy = (xh - xl) / M, (yh - yl) / N
    px = rng.uniform(xl - 5, xh + 1, n).astype(np.float32).astype(np.float64)
    py = rng.uniform(yl - 5, yh + 1, n).astype(np.float32).astype(np.float64)
    sx = rng.uniform(0.2, 3.0, n) * bsx
    sy = rng.uniform(0.2, 2.5, n) * bsy
    sx[:3] = [0.0, -1.0, 70.0]       # zero, negative, wider than the die
    px[2] = xl - 10.0
    px[3] = xl + 2 * bsx             # exactly on a bin edge
    sx[3] = bsx
    sx = sx.astype(np.float32).astype(np.float64)
    sy = sy.astype(np.float32).astype(np.float64)
    out.update(px=px, py=py, sx=sx, sy=sy, geom=np.array([M, N, xl, yl, xh, yh]))
    out["rho_stretch"] = loop_density(px, py, sx, sy, M, N, xl, yl, xh, yh, True)
    out["rho_nostretch"] = loop_density(px, py, sx, sy, M, N, xl, yl, xh, yh, False)
    np.savez_compressed(os.path.join(HERE, "density_golden.npz"), **out)


if __name__ == "__main__":
    spectral()
    density()
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))
