"""Page router with the tiers of the reference runtime, on the HIP library.

``route`` returns ``(ids, mask, risk, stats)`` like the reference's
``BatchGraphs.replay`` (reproduction/vbench_current/graph.py:212-221):

* ``tier='base'``: ids = [own, anchors 0..23, the floor(0.15 P) - 25 highest-
  risk other pages] (local_experiments/video_runtime_v1/runtime.py:279-288).
* ``tier='intersection'``: anchors + top A current pages (own forced) + top
  (n - A) history pages; ids = own first then descending risk
  (reproduction/vbench_current/quota_mask.py:7-39, graph.py:150-151,210).
  Quotas larger than their partition keep the whole partition and the table
  is padded with -1.  A 72-page window (the anchor frame is the chunk's first
  frame, graph.py:143-148) keeps the anchors and the top n of pages 24..71.
* ``tier='topk'``: fixed top-floor(0.1 P) with own forced
  (local_experiments/review_v1/ops.py:113-138).

With ``full_pset`` heads (intersection tier), the Full_Pset swap correction
runs on those heads after selection and rewrites their mask and ids
(reproduction/vbench_current/graph.py:169-210); ``stats`` is then
(executed swaps, corrected rows, non-finite scores).

Probe rows are read straight from q (16 per 64-query block at the reference's
offsets, local_experiments/video_runtime_v1/runtime.py:84).
"""
from __future__ import annotations

import math

import torch

from . import _lib
from .legacy_components import HEAD_DIM, _check_summary, check_rep_ops

ANCHORS = 24
CURRENT = 72
MODES = {'base': 0, 'intersection': 1, 'topk': 2}


def tier_count(tier: str, pages: int, n: int | None = None) -> int:
    if tier == 'base':
        return pages * 15 // 100
    if tier == 'intersection':
        return ANCHORS + int(n)
    if tier == 'topk':
        return max(1, int(pages * 0.1))
    raise ValueError(tier)


@torch.no_grad()
def route(q, summary, theta, *, tier='base', own=None, current_slots=None, n=None, workspace=None,
          want_mask=True, full_pset=None, encoding=None, reader=None, lse_out=None, rep_out=None, ties=None,
          tie_eps=1e-3):
    """q [1,N,H,128] bf16 queries of the current chunk; summary over the P
    window pages; theta [H,4]; own [H,T] (default: page P-T+t).  For the
    intersection tier pass n = A+B (<= P - 24) and, unless P == 72,
    current_slots [H] (A per head).
    full_pset: head ids to correct with `encoding` (pset.Encoding over the
    window) and `reader` (pset.Reader).  lse_out: optional [H,T,16] fp32
    tensor that receives each probe's log-sum-exp over all reps.
    rep_out [H,>=ceil(P/16),512] bf16: the router also writes the
    attention's detail operand tiles of `summary` (as
    legacy_components.rep_operands) into rep_out, so attention(...,
    rep_ops=rep_out) skips that launch.
    ties: optional (rows [H*T] int32, count [1] int32) device tensors that
    receive the rows h*T + t whose selection boundary is a near tie (last
    kept and first dropped risk within tie_eps relative; own never counts)
    and their number, as the reference's select_close reports them for its
    recheck; they describe the router's selection, before any Full_Pset
    swap."""
    _, nq, h, d = q.shape
    if d != HEAD_DIM or q.dtype != torch.bfloat16 or not q.is_contiguous():
        raise ValueError("q must be contiguous [1,N,H,128] bf16")
    t = nq // 64
    p = summary.mean.shape[1]
    hp = _check_summary(summary, h, p)
    if tier not in MODES:
        raise ValueError(f"unknown tier {tier!r}")
    if tier == 'intersection' and (n is None or (current_slots is None and p != CURRENT)):
        raise ValueError("intersection tier needs n and (unless P == 72) current_slots")
    if tier == 'intersection' and not 0 <= int(n) <= p - ANCHORS:
        raise ValueError(f"intersection quota n={n} outside [0, P-24]")
    mode = MODES[tier]
    count = tier_count(tier, p, n)
    dev = q.device
    cur = None
    total = 0
    if tier == 'intersection':
        if current_slots is not None:
            cur = torch.as_tensor(current_slots, device=dev).to(torch.int32).contiguous()
            if cur.shape != (h,):
                raise ValueError("current_slots must be [H]")
        total = int(n)
    if tier == 'base' and p < ANCHORS + CURRENT:
        raise ValueError("base tier needs a history window")
    correcting = full_pset is not None and len(full_pset) > 0
    if correcting:
        if tier != 'intersection' or encoding is None or reader is None:
            raise ValueError("full_pset needs the intersection tier, an encoding and a reader")
        want_mask = True

    def buf(name, shape, dtype):
        if workspace is None:
            return torch.empty(shape, device=dev, dtype=dtype)
        return workspace.tensor('route_' + name, shape, dev, dtype)

    ow = None
    if own is not None:
        ow = own if (own.dtype == torch.int32 and own.is_contiguous()) else own.to(device=dev, dtype=torch.int32).contiguous()
    risk = buf('risk', (h, t, p), torch.float32)
    ids = buf('ids', (h, t, count), torch.int32)
    mask = buf('mask', (h, t, p), torch.uint8) if want_mask else None
    th = theta.float().contiguous()
    lse = lse_out
    if lse is None and correcting:
        lse = buf('lse', (h, t, 16), torch.float32)
    if lse is not None and (lse.shape != (h, t, 16) or lse.dtype != torch.float32 or not lse.is_contiguous()):
        raise ValueError("lse_out must be a contiguous [H,T,16] float32 tensor")
    if rep_out is not None:
        check_rep_ops(rep_out, h, p, "rep_out")
    tie_rows = tie_count = None
    if ties is not None:
        tie_rows, tie_count = ties
        if tie_rows.dtype != torch.int32 or tie_rows.numel() < h * t or not tie_rows.is_contiguous() or \
                tie_count.dtype != torch.int32 or tie_count.numel() < 1:
            raise ValueError("ties must be (rows int32 [>=H*T], count int32 [1]) device tensors")
        if not tie_eps >= 0:
            raise ValueError("tie_eps must be >= 0")
    _lib.check(_lib.lib().ssa_route(_lib.ptr(q), d, 64 * h * d, h * d, 0, _lib.ptr(summary.keys),
                                    _lib.ptr(summary.stats), _lib.ptr(th), _lib.ptr(cur), _lib.ptr(ow),
                                    _lib.ptr(risk), _lib.ptr(ids), _lib.ptr(mask), _lib.ptr(lse), h, t, p, hp, count,
                                    mode, total, _lib.ptr(summary.detail) if rep_out is not None else None,
                                    _lib.ptr(rep_out), rep_out.shape[1] if rep_out is not None else 0,
                                    float(tie_eps), _lib.ptr(tie_rows), _lib.ptr(tie_count),
                                    _lib.stream_handle(dev)), "ssa_route")
    if correcting:
        from . import pset
        stats, _ = pset.correct(q, summary, encoding, reader, risk, lse, mask, ids, ow, full_pset, workspace)
    elif workspace is None:
        stats = torch.zeros(3, device=dev, dtype=torch.int64)
    else:
        key = ('route_stats', (3,), torch.device(dev), torch.int64)
        if key not in workspace.entries:
            workspace.entries[key] = torch.zeros(3, device=dev, dtype=torch.int64)
        stats = workspace.entries[key]
    # uint8 0/1 storage viewed as bool without a conversion kernel
    return ids, (mask.view(torch.bool) if mask is not None else None), risk, stats


@torch.no_grad()
def select(scores, own, config=None, threshold=None, valid=None, *, density=0.10, max_fraction=0.25,
           id_capacity=128):
    """RouteOps.select (local_experiments/review_v1/ops.py:113-138) on the HIP
    library: scores [H,T,P] (a page risk), own [H,T] (one protected page per
    row), `config` any object with density / max_fraction / id_capacity (the
    reference's Config; keyword defaults otherwise), optional threshold and
    valid [H,T,P] bool.  Returns dict(ids [H,T,id_capacity] int32 with -1
    padding, counts [H,T] int32, mask [H,T,P] bool, overflow [H,T] int32,
    residual_risk [H,T] fp32) as the reference does."""
    if config is not None:
        density, max_fraction, id_capacity = config.density, config.max_fraction, config.id_capacity
    h, t, p = scores.shape
    if not 0 < density <= max_fraction <= 1 or id_capacity < math.ceil(max_fraction * p):
        raise ValueError("need 0 < density <= max_fraction <= 1 and id_capacity >= ceil(max_fraction * P)")
    if p > 512:
        raise ValueError("at most 512 pages")
    dev = scores.device
    sc = scores.float().contiguous()
    ow = own.to(device=dev, dtype=torch.int32).expand(h, t).contiguous()
    vd = None
    if valid is not None:
        vd = valid.expand(h, t, p).to(device=dev, dtype=torch.uint8).contiguous()
    cap = min(id_capacity, math.ceil(max_fraction * p))
    fixed = max(1, math.floor(p * density))
    ids = torch.empty(h, t, id_capacity, device=dev, dtype=torch.int32)
    counts = torch.empty(h, t, device=dev, dtype=torch.int32)
    mask = torch.empty(h, t, p, device=dev, dtype=torch.uint8)
    overflow = torch.empty(h, t, device=dev, dtype=torch.int32)
    residual = torch.empty(h, t, device=dev, dtype=torch.float32)
    thr = 0.0 if threshold is None else float(threshold)
    _lib.check(_lib.lib().ssa_select(_lib.ptr(sc), _lib.ptr(ow), _lib.ptr(vd), h * t, p, thr,
                                     int(threshold is not None), fixed, cap, id_capacity, _lib.ptr(ids),
                                     _lib.ptr(counts), _lib.ptr(mask), _lib.ptr(overflow), _lib.ptr(residual),
                                     _lib.stream_handle(dev)), "ssa_select")
    return dict(ids=ids, counts=counts, mask=mask.view(torch.bool), overflow=overflow, residual_risk=residual)

