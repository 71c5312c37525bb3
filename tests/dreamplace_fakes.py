"""Stand-ins for what DREAMPlace hands ElectricPotentialFunction.forward, for
tests of the adapter without DREAMPlace (which is not importable here):

  * forward_args(): the positional arguments of the patched forward
    (reference integration/scatter_ttnn_client.py:553-574) for a set of
    movable cells, fixed terminals and fillers, laid out as DREAMPlace lays
    out pos ([movable | terminals | filler], :611-617), with clamped sizes and
    offsets as DREAMPlace computes them (size = clamped + 2 * offset);
  * Transforms: dct2 / idxst_idct / idct_idxst objects with .forward and the
    wu/wv weight maps, as dense matrices in the conventions of the reference
    server's TTNN solver (host/density_scatter_ttnn_server_host.cpp:124-181,
    :251-263, :281-295), so the CPU_DCT chain the adapter runs can be checked
    against the oracle's fields.  DREAMPlace's own normalisation of these
    operators is not pinned here.
"""
import numpy as np


class Ctx:
    """The autograd context object the forward stashes its state in."""


def _mats(K):
    k = np.arange(K)[:, None]
    n = np.arange(K)[None, :]
    C = (2.0 / K) * np.cos(np.pi * k * (n + 0.5) / K)          # DCT-II rows
    Ik = 2.0 * np.cos(np.pi * n * (k + 0.5) / K)
    Ik[:, 0] = 1.0                                             # I_K[k, 0] = 1
    S = np.sin(np.pi * n * (k + 0.5) / K)
    return C, Ik, S


class _Op:
    def __init__(self, left, right):
        import torch
        self.left = torch.from_numpy(left)
        self.right = torch.from_numpy(right)

    def forward(self, x):
        x = x.to(self.left.dtype)
        return self.left @ x @ self.right.T


class Transforms:
    def __init__(self, M, N, bsx, bsy):
        import torch
        CM, IM, SM = _mats(M)
        CN, IN, SN = _mats(N)
        self.dct2 = _Op(CM, CN)
        self.idxst_idct = _Op(2.0 * SM, IN)
        self.idct_idxst = _Op(2.0 * IM, SN)
        wu = (2.0 * np.pi * np.arange(M) / M)[:, None]
        wv = (2.0 * np.pi * np.arange(N) / N * (bsx / bsy))[None, :]
        D = wu * wu + wv * wv
        D[0, 0] = 1.0
        wx, wy = wu / (2.0 * D), wv / (2.0 * D)
        wx[0, 0] = wy[0, 0] = 0.0
        self.wu_by = torch.from_numpy(wx)
        self.wv_by = torch.from_numpy(wy)


def forward_args(mov, term, fil, M, N, die, d0n, transforms=None, dtype=None):
    """mov, term, fil: (px, py, sx, sy) arrays of movable cells, fixed
    terminals and fillers; die = (xl, yl, xh, yh); d0n = initial density /
    bin area (M x N).  Returns (args, sel) where args follow ctx in the
    forward's signature and sel maps the scattered cells ([movable | filler])
    to their index in each coordinate half of pos."""
    import torch
    dtype = dtype or torch.float64
    xl, yl, xh, yh = die
    bsx, bsy = (xh - xl) / M, (yh - yl) / N
    parts = [np.asarray(p, np.float64) for p in (mov, term, fil)]
    px = np.concatenate([p[0] for p in parts])
    py = np.concatenate([p[1] for p in parts])
    sx = np.concatenate([p[2] for p in parts])
    sy = np.concatenate([p[3] for p in parts])
    n_mov, n_term, n_fil = (len(p[0]) for p in parts)
    n = n_mov + n_term + n_fil
    # DREAMPlace clamps small cells to sqrt2 * bin and keeps the offset
    csx = np.maximum(sx, np.sqrt(2.0) * bsx)
    csy = np.maximum(sy, np.sqrt(2.0) * bsy)
    t = lambda a: torch.from_numpy(np.asarray(a, np.float64)).to(dtype)
    pos = t(np.concatenate([px, py]))
    init = t(np.asarray(d0n, np.float64).reshape(M, N) * (bsx * bsy))
    tf = transforms
    args = (pos, t(csx), t(csy), t((sx - csx) / 2), t((sy - csy) / 2),
            t((sx * sy) / (csx * csy)), None, None, init, 1.0, xl, yl, xh, yh,
            bsx, bsy, n_mov, n_fil, 0, None, M, N, 0, 0, 0, 0, True, None,
            None, None, None,
            tf.wu_by if tf else None, tf.wv_by if tf else None,
            tf.dct2 if tf else None, None,
            tf.idct_idxst if tf else None, tf.idxst_idct if tf else None)
    sel = np.r_[0:n_mov, n - n_fil:n]
    return args, sel
