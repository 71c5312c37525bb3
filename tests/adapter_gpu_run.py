"""Child process of tests/test_gpu_server.py::test_dreamplace_adapter_forces_on_gpu.

Drives the DREAMPlace adapter (make_forward / make_backward) through the shm
server on the 1.1M-cell, 2048 x 2048 workload (seed 0), with the last tenth of
the cells as fillers and 64 fixed terminals between them in pos, float32 as
DREAMPlace runs, and compares the backward's gradient and the stashed field
maps with the float64 oracle.  A second iteration moves the cells: the
adapter then sends the positions alone (the size tensors are unchanged) and
its gradient is checked the same way.  Prints one JSON line of relative
errors.

    python adapter_gpu_run.py IPC_DIR
"""
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
for p in (HERE, os.path.join(ROOT, "dreamplacett-framework_amd"), os.path.join(ROOT, "oracle")):
    sys.path.insert(0, p)

import numpy as np  # noqa: E402
import torch  # noqa: E402

import dreamplace_fakes as F  # noqa: E402
import pyoracle  # noqa: E402
from dpep import scatter_ttnn_client as stc  # noqa: E402
from dpep import workloads  # noqa: E402


def rel_l2(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(np.linalg.norm(a - b) / (np.linalg.norm(b) or 1.0))


def main():
    ipc = sys.argv[1]
    w = workloads.make(3, seed=0)
    px, py, sx, sy = w.cells(np.float32)
    n = w.nc
    nf = n // 10
    rng = np.random.default_rng(7)
    term = (rng.uniform(w.xl, w.xh - 2000, 64), rng.uniform(w.yl, w.yh - 2000, 64),
            rng.uniform(300, 2000, 64), rng.uniform(300, 2000, 64))
    mov = (px[:n - nf], py[:n - nf], sx[:n - nf], sy[:n - nf])
    fil = (px[n - nf:], py[n - nf:], sx[n - nf:], sy[n - nf:])
    die = (w.xl, w.yl, w.xh, w.yh)
    args, sel = F.forward_args(mov, term, fil, w.M, w.N, die, w.d0n, dtype=torch.float32)
    print(f"adapter: {len(sel)} scattered cells, 64 terminals, {w.M}x{w.N}", flush=True)

    client = stc.ScatterTTNNClient(ipc_dir=ipc, nc_max=len(sel), as_torch=False,
                                   ready_timeout=300, step_timeout=120)
    fwd = stc.make_forward(client, keep_field_maps=True).__func__
    bwd = stc.make_backward().__func__
    steps = []
    try:
        for it in range(2):
            if it == 1:     # cells move; the size tensors stay as they were
                args[0].add_(torch.from_numpy(
                    rng.normal(0, 20, args[0].numel()).astype(np.float32)))
            ctx = F.Ctx()
            fwd(ctx, *args)
            grad = bwd(ctx, torch.tensor([0.5], dtype=torch.float32))[0].numpy()
            word = int(np.frombuffer(client._mm, np.uint32, 1, stc.S.OFF_OUTPUTS)[0])
            steps.append((args[0].numpy().copy(), grad, ctx,
                          bool(word & stc.S.IN_KEEP_SIZES)))
            print(f"adapter iteration {it} timing",
                  {k: round(v, 3) for k, v in client._timings[-1].items()
                   if isinstance(v, float)}, flush=True)
    finally:
        client.stop()

    # the cells exactly as the adapter sent them (sizes = clamped + 2 offset
    # in float32)
    osx = (args[1] + 2.0 * args[3]).numpy()
    osy = (args[2] + 2.0 * args[4]).numpy()
    res = {}
    for it, (pos, grad, ctx, kept) in enumerate(steps):
        half = pos.size // 2
        cells = (pos[:half][sel], pos[half:][sel], osx[sel], osy[sel])
        ref = pyoracle.step(*cells, w.M, w.N, *die, d0n=w.d0n.astype(np.float32))
        term_idx = np.setdiff1d(np.arange(half), sel)
        sfx = "" if it == 0 else "_moved"
        res["grad_x" + sfx] = rel_l2(grad[:half][sel], -0.5 * ref["grad_x"])
        res["grad_y" + sfx] = rel_l2(grad[half:][sel], -0.5 * ref["grad_y"])
        res["field_x" + sfx] = rel_l2(ctx.field_map_x.numpy(), ref["field_x"])
        res["field_y" + sfx] = rel_l2(ctx.field_map_y.numpy(), ref["field_y"])
        res["terminals_zero" + sfx] = bool(np.all(grad[:half][term_idx] == 0) and
                                           np.all(grad[half:][term_idx] == 0))
        res["sizes_kept" + sfx] = kept
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
