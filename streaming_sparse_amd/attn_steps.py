"""Per-step time of the one-block attention kernel, from the measurement build.

    python -m streaming_sparse_amd.build --stamps
    python -m streaming_sparse_amd.attn_steps [--single-av]

The measurement build (libssattn_stamps.so, the same sources compiled with
-DSSA_ROUTE_STAMPS and -DSSA_ATTN_STAMPS) has lane 0 of every attention wave
record the shader clock (s_memtime) at the kernel's phase boundaries and at
three points of every paired step: its start (after the previous barrier),
the end of its body (loads issued, matrix products, softmax, running-max
update) and the end of its wait for the step's own loads; the next step's
start closes the barrier.  This module runs the base-tier call at 432 pages
(12 heads x 4608 queries, 64 exact pages per block) through that library
after a warm-up, reads the stamps of the last attention launch
(ssa_attn_stamps) and prints, in shader cycles:

* per wave of a whole tile, the phases of the kernel;
* per paired step, mean and percentiles of body, load wait and barrier, for
  page steps (unit i an exact page) and rep steps (unit i a rep tile), each
  split by whether another workgroup shared the CU for the whole step.

The clock counts per XCD, so only differences within one XCD are used; the
workgroups sharing a CU are found from the HW_ID and XCC_ID stamps.  Each
stamp costs its wave a clock read and an LDS write (the step-start one waits
for the read), so the measurement build runs somewhat slower than the
product library; the launch time of both is printed.
"""
from __future__ import annotations

import argparse
import collections
import time

import numpy as np
import torch

from . import _lib, build, workload
from .attention import Workspace
from .legacy_components import REP_OP_ELEMS, attention, rep_tiles
from .route import route

WGS, REC, HEAD = 1024, 296, 8


def launch_ms(fn, n=100):
    """Median event time of `fn` over n calls (ms)."""
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    for a, b in ev:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    return float(np.median([a.elapsed_time(b) for a, b in ev]))


def read_stamps():
    buf = np.zeros(WGS * 4 * REC, dtype=np.uint64)
    _lib.check(_lib.lib().ssa_attn_stamps(buf.ctypes.data, buf.nbytes), "ssa_attn_stamps")
    return buf.reshape(WGS, 4, REC)


def summarize(st, wgs, split_from):
    """Phase and step statistics of the first `wgs` workgroups' stamps."""
    st = st[:wgs].astype(np.int64)
    info = st[:, :, 6]
    npages = (info & 0xffff)[:, 0]
    ibeg = ((info >> 32) & 0xffff)[:, 0]
    iend_pair = ((info >> 48) & 0xffff)[:, 0]
    hw = st[:, 0, 7]
    cu = ((hw >> 32) & 0xff) * 4096 + (hw & 0xffff) // 256   # XCC, then the CU/SH/SE bits of HW_ID
    start, end = st[:, :, 0].min(1), st[:, :, 5].max(1)
    # workgroup intervals per CU, to tell whether a step had the CU to itself
    by_cu = collections.defaultdict(list)
    for g in range(wgs):
        by_cu[int(cu[g])].append(g)

    def shared(g, t0, t1):
        return any(o != g and start[o] <= t0 and end[o] >= t1 for o in by_cu[int(cu[g])])

    phases = {"start -> unit list built": (0, 1), "unit list -> prologue done": (1, 2),
              "paired steps": (2, 3), "last units": (3, 4), "key halves exchanged": (4, 5)}
    whole = [g for g in range(wgs) if g < split_from]
    print(f"per wave of a whole tile, cycles (mean / max over {4 * len(whole)} waves):")
    for label, (a, b) in phases.items():
        d = st[whole, :, b] - st[whole, :, a]
        print(f"  {label:40s} {d.mean():9.0f} {d.max():9.0f}")
    d = st[whole, :, 5] - st[whole, :, 0]
    print(f"  {'total':40s} {d.mean():9.0f} {d.max():9.0f}")
    rows = collections.defaultdict(list)   # (kind, shared) -> [(body, wait, barrier)]
    for g in whole:
        n = int(min(iend_pair[g] - ibeg[g], (REC - HEAD) // 3))
        for w in range(4):
            t = st[g, w, HEAD:HEAD + 3 * n].reshape(n, 3)
            nxt = np.append(t[1:, 0], st[g, w, 3])
            for k in range(n):
                kind = "page" if ibeg[g] + k < npages[g] else "rep"
                sh = shared(g, t[k, 0], nxt[k])
                rows[(kind, sh)].append((t[k, 1] - t[k, 0], t[k, 2] - t[k, 1], nxt[k] - t[k, 2]))
    print("per paired step, cycles: mean (p10 / p50 / p90)")
    for kind in ("page", "rep"):
        for sh in (True, False):
            a = np.array(rows[(kind, sh)], dtype=np.float64)
            if len(a) == 0:
                continue
            tot = a.sum(1)
            label = f"{kind} steps, CU {'shared' if sh else 'alone'} ({len(a)} wave-steps)"
            print(f"  {label}")
            for name, col in (("body", a[:, 0]), ("own loads wait", a[:, 1]), ("barrier", a[:, 2]),
                              ("step", tot)):
                p10, p50, p90 = np.percentile(col, [10, 50, 90])
                print(f"    {name:18s} {col.mean():8.0f} ({p10:6.0f} / {p50:6.0f} / {p90:6.0f})")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--single-av", action="store_true", help="single-term bf16 P.V")
    args = ap.parse_args()
    dev = torch.device("cuda:0")
    x = workload.make_call(cfg=1, frames=18).to(dev)
    P, H = x.pages, 12
    ws = Workspace()
    ops = ws.tensor('ops', (H, rep_tiles(P), REP_OP_ELEMS), dev, torch.bfloat16)
    basis = x.basis.to(torch.bfloat16).contiguous()
    ids, _, _, _ = route(x.q, x.summary, x.theta, tier='base', workspace=ws, want_mask=False, rep_out=ops)
    call = lambda: attention(x.q, x.k, x.v, x.summary, basis, ids, ws, single_av=args.single_av, rep_ops=ops)
    t0 = time.time()
    while time.time() - t0 < 0.3:
        call()
    product_ms = launch_ms(call)
    _lib.use(build.STAMPS_LIB)
    t0 = time.time()
    while time.time() - t0 < 0.3:
        call()
    stamps_ms = launch_ms(call)
    call()
    torch.cuda.synchronize()
    st = read_stamps()
    tiles = H * (x.q.shape[1] // 64)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    split = tiles % cus
    split_from = tiles - split
    print(f"attention call ({'single' if args.single_av else 'two'}-term P.V, {tiles} tiles: {split_from} whole + "
          f"{split} in 2 pieces): {product_ms * 1e3:.1f} us per call with the product library, "
          f"{stamps_ms * 1e3:.1f} us with the measurement build")
    summarize(st, split_from + 2 * split, split_from)


if __name__ == "__main__":
    main()
