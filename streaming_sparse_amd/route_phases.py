"""Per-phase time of the router kernel, from the measurement build.

    python -m streaming_sparse_amd.build --stamps
    python -m streaming_sparse_amd.route_phases

The measurement build (libssattn_stamps.so, the same sources compiled with
-DSSA_ROUTE_STAMPS and -DSSA_ATTN_STAMPS) has lane 0 of every router wave record the shader clock
at the kernel's phase boundaries.  This module runs the full-window base and
intersection calls (12 heads x 4608 queries, 432 pages) through that library
after a warm-up, reads the stamps of the last launch (ssa_route_stamps) and
prints, per phase, the mean and the maximum over the 1,728 router waves of
the cycles between its two stamps.  The clock counts per XCD, so only
differences within one wave are used.
"""
from __future__ import annotations

import time

import numpy as np
import torch

from . import _lib, build, workload
from .attention import Workspace
from .legacy_components import REP_OP_ELEMS, rep_tiles
from .route import route

PHASES = ("setup loads (probes, stats maximum inputs, theta, own)", "setup arithmetic (probe norms, operands, first tiles issued)",
          "rep tiles (logits, risk features)", "probe totals", "page values into LDS", "probe sums, risk rows",
          "sort keys", "bitonic sort", "sorted keys to LDS", "table, near-tie report, mask")
BLOCKS, SLOTS = 1024, 16


def phases(call, router_blocks):
    """Mean and max cycles per phase over the router waves of `call`'s last launch."""
    buf = np.zeros(BLOCKS * 4 * SLOTS, dtype=np.uint64)
    call()
    torch.cuda.synchronize()
    _lib.check(_lib.lib().ssa_route_stamps(buf.ctypes.data, buf.nbytes), "ssa_route_stamps")
    st = buf.reshape(BLOCKS * 4, SLOTS)[: router_blocks * 4, : len(PHASES) + 1].astype(np.int64)
    d = np.diff(st, axis=1)
    tot = st[:, -1] - st[:, 0]
    return d.mean(0), d.max(0), tot.mean(), tot.max()


def main():
    _lib.use(build.STAMPS_LIB)
    dev = torch.device("cuda:0")
    x = workload.make_call(cfg=1, frames=18).to(dev)
    P = x.pages
    ws = Workspace()
    ops = ws.tensor('ops', (12, rep_tiles(P), REP_OP_ELEMS), dev, torch.bfloat16)
    cur = torch.full((12,), 18, dtype=torch.int32, device=dev)
    calls = {
        "base (own + 24 anchors + 39 by risk, operand tiles on the side)":
            lambda: route(x.q, x.summary, x.theta, tier='base', workspace=ws, want_mask=False, rep_out=ops),
        "intersection (A = 18 current, B = 26 history)":
            lambda: route(x.q, x.summary, x.theta, tier='intersection', n=44, current_slots=cur, workspace=ws),
    }
    router_blocks = 12 * 36
    for name, call in calls.items():
        t0 = time.time()
        while time.time() - t0 < 0.3:
            call()
        mean, mx, tmean, tmax = phases(call, router_blocks)
        print(f"{name}: cycles per router wave (mean / max over {router_blocks * 4} waves)")
        for label, a, b in zip(PHASES, mean, mx):
            print(f"  {label:60s} {a:8.0f} {b:8.0f}")
        print(f"  {'total':60s} {tmean:8.0f} {tmax:8.0f}")


if __name__ == "__main__":
    main()
