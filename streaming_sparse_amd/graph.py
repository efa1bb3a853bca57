"""Route graphs with the reference's call shape, on the HIP library.

Mirrors BatchGraphs of reproduction/vbench_current/graph.py (:20-93 get and
stage, :212-221 replay): ``get(q, summary, encoding, theta, basis, own,
full_pset, heads)`` prepares one call shape -- static input buffers, the
route outputs and a captured HIP graph of the route (probe logits, risk,
selection and page table in one ssa_route launch that also writes the
compensation's detail operand tiles, then, with full_pset, the ssa_pset swap
correction of the scoped heads) -- and ``replay(e, q, own)`` copies the query
batch and own pages into the entry and replays the graph, returning
``(ids, mask, risk, stats)``.

As in the reference, the caller sets ``n`` (A + B, the table width 24 + n is
part of an entry's key) and ``current_slots`` (A per head) before each
``get``, the way queue_policy.attach does (VB/queue_policy.py:25-33);
current_slots is read again on every replay.

``q`` has the reference's block layout [H, T, n, D] (VB/graph.py:103-105):
n = 64, the block's queries, whose probe rows are rows round(63 m / 15); or
n = 16, the probe rows themselves (its input_m16 mode).  The attention call
that follows takes the entry's ``rep_ops`` (legacy_components.attention(...,
rep_ops=e['rep_ops'])).
"""
from __future__ import annotations

import torch

from . import _lib, pset
from .attention import Workspace
from .legacy_components import HEAD_DIM, REP_OP_ELEMS, _check_summary, rep_tiles
from .ops import Summary
from .route import ANCHORS, CURRENT, MODES, tier_count


class BatchGraphs:
    """Captured route graphs keyed by call shape.  tier: 'intersection' (the
    reference's anchor policy, VB/quota_mask.py), 'base' (VR/runtime.py:279-
    288) or 'topk' (RouteOps.select at density 0.1).  reader: the Full_Pset
    pset.Reader (the reference's phi).  capture=False replays by running the
    launches eagerly (the reference's inline mode)."""

    def __init__(self, tier='intersection', reader=None, capture=True):
        if tier not in MODES:
            raise ValueError(f"unknown tier {tier!r}")
        self.tier = tier
        self.reader = reader
        self.capture = capture
        self.n = None                 # A + B, set per call (intersection tier)
        self.current_slots = None     # [H] device tensor of A, set per call
        self.entries = {}
        self.calls = 0
        self.pool = None

    # --------------------------------------------------------------- get --

    @torch.no_grad()
    def get(self, q, summary: Summary, encoding, theta, basis, own, full_pset, heads=None, resident=False):
        h, t, n, d = q.shape
        p = summary.mean.shape[1]
        if d != HEAD_DIM or n not in (16, 64):
            raise ValueError("q must be [H, T, 64 or 16, 128]")
        if self.tier == 'intersection' and (self.n is None or (self.current_slots is None and p != CURRENT)):
            raise ValueError("set n (and, unless P == 72, current_slots) before get, as attach does")
        scoped = None
        if full_pset:
            if heads is None or self.reader is None or encoding is None or self.tier != 'intersection':
                raise ValueError("full_pset needs the intersection tier, heads, an encoding and the reader")
            scoped = [int(i) for i in (heads.tolist() if torch.is_tensor(heads) else heads)]
            if not scoped or len(set(scoped)) != len(scoped) or min(scoped) < 0 or max(scoped) >= h:
                raise ValueError(f"full_pset heads must be distinct ids in [0,{h})")
        key = (h, t, p, bool(full_pset), q.device, n, 0 if scoped is None else len(scoped),
               self.n if self.tier == 'intersection' else None)
        if resident:
            key += ('resident', summary.keys.data_ptr(), summary.stats.data_ptr())
        if key not in self.entries:
            self.entries[key] = self._build(q, summary, encoding, theta, basis, own, full_pset, scoped, resident)
        e = self.entries[key]
        if scoped is not None:
            e['heads'].copy_(torch.tensor(scoped, dtype=torch.int32))
        if not resident:
            self.stage(e, summary, encoding, theta, basis)
        return e

    def _build(self, q, summary, encoding, theta, basis, own, full_pset, scoped, resident):
        h, t, n, d = q.shape
        p = summary.mean.shape[1]
        dev = q.device
        hp = _check_summary(summary, h, p)
        count = tier_count(self.tier, p, self.n)
        e = dict(full_pset=bool(full_pset), resident=resident, n=self.n, count=count, pages=p)
        e['q'] = torch.empty(h, t, n, d, device=dev, dtype=torch.bfloat16)
        e['own'] = torch.empty(h, t, device=dev, dtype=torch.int32)
        e['theta'] = torch.empty(h, 4, device=dev, dtype=torch.float32)
        if resident:
            e['s'], e['basis'], e['en'] = summary, basis, encoding
        else:
            e['s'] = Summary(*(torch.empty_like(getattr(summary, f)) for f in Summary.FIELDS))
            e['basis'] = torch.empty(h, d, 8, device=dev, dtype=torch.bfloat16)
            e['en'] = None if encoding is None else pset.Encoding(*(torch.empty_like(x) for x in (
                encoding.coef, encoding.mean, encoding.detail)))
        e['current'] = torch.zeros(h, device=dev, dtype=torch.int32)
        e['heads'] = torch.zeros(0 if scoped is None else len(scoped), device=dev, dtype=torch.int32)
        e['risk'] = torch.empty(h, t, p, device=dev, dtype=torch.float32)
        e['ids'] = torch.empty(h, t, count, device=dev, dtype=torch.int32)
        e['mask'] = torch.empty(h, t, p, device=dev, dtype=torch.uint8)
        e['lse'] = torch.empty(h, t, 16, device=dev, dtype=torch.float32)
        e['stats'] = torch.zeros(3, device=dev, dtype=torch.int64)
        e['rep_ops'] = torch.empty(h, rep_tiles(p), REP_OP_ELEMS, device=dev, dtype=torch.bfloat16)
        e['ws'] = Workspace()
        e['hp'] = hp
        # the probe rows: [H, T, 64, D] blocks (rows at the reference offsets) or [H, T, 16, D] probes
        e['layout'] = (t * n * d, n * d, d, 1 if n == 16 else 0)
        if not resident:
            self.stage(e, summary, encoding, theta, basis)
        else:
            e['theta'].copy_(theta)
        e['q'].copy_(q)
        e['own'].copy_(own)
        if self.current_slots is not None:
            e['current'].copy_(self.current_slots)
        if scoped is not None:
            e['heads'].copy_(torch.tensor(scoped, dtype=torch.int32))
        # warm-up launches on a side stream, then the capture (VB/graph.py:75-80)
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(3):
                self.compute(e)
        torch.cuda.current_stream(dev).wait_stream(side)
        e['graph'] = None
        if self.capture:
            if self.pool is None:
                self.pool = torch.cuda.graph_pool_handle()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, pool=self.pool):
                self.compute(e)
            graph.replay()
            e['graph'] = graph
        return e

    @torch.no_grad()
    def stage(self, e, s, encoding, theta, basis):
        """Copy the layer's page data into the entry (VB/graph.py:82-89)."""
        for f in Summary.FIELDS:
            getattr(e['s'], f).copy_(getattr(s, f))
        if e['en'] is not None and encoding is not None:
            for x, y in zip((e['en'].coef, e['en'].mean, e['en'].detail),
                            (encoding.coef, encoding.mean, encoding.detail)):
                x.copy_(y)
        e['theta'].copy_(theta)
        e['basis'].copy_(basis)

    # ----------------------------------------------------------- compute --

    def compute(self, e):
        """The route of one entry: ssa_route (risk, mask, page table, probe
        log-sum-exp and the detail operand tiles), then with full_pset the
        ssa_pset correction of the scoped heads, which rewrites mask and ids
        in place and writes the stats."""
        q, s = e['q'], e['s']
        h, t, _, _ = q.shape
        p = e['pages']
        stream = _lib.stream_handle(q.device)
        current = e['current'] if self.tier == 'intersection' and p != CURRENT else None
        _lib.check(_lib.lib().ssa_route(
            _lib.ptr(q), *e['layout'], _lib.ptr(s.keys), _lib.ptr(s.stats), _lib.ptr(e['theta']),
            _lib.ptr(current), _lib.ptr(e['own']), _lib.ptr(e['risk']), _lib.ptr(e['ids']), _lib.ptr(e['mask']),
            _lib.ptr(e['lse']), h, t, p, e['hp'], e['count'], MODES[self.tier],
            int(e['n']) if self.tier == 'intersection' else 0, _lib.ptr(s.detail), _lib.ptr(e['rep_ops']),
            e['rep_ops'].shape[1], 0.0, None, None, stream), "ssa_route")
        if e['full_pset']:
            # the entry's device head list and its own scratch, so the captured launches read both
            stats, _ = pset.correct(q, s, e['en'], self.reader, e['risk'], e['lse'], e['mask'], e['ids'],
                                    e['own'], e['heads'], e['ws'], probe_layout=e['layout'])
            e['stats'] = stats
        return e['ids'], e['mask'], e['risk'], e['stats']

    # ------------------------------------------------------------ replay --

    @torch.no_grad()
    def replay(self, e, q, own):
        """Copy the query batch and own pages into the entry if they are other
        tensors, re-read current_slots, and replay the entry's graph (or run
        its launches when capture is off or a capture is in progress)."""
        if e['q'] is not q:
            e['q'].copy_(q)
        if e['own'] is not own:
            e['own'].copy_(own)
        if self.current_slots is not None and self.tier == 'intersection':
            e['current'].copy_(self.current_slots)
        if e['graph'] is None or torch.cuda.is_current_stream_capturing():
            self.compute(e)
        else:
            e['graph'].replay()
        self.calls += 1
        return e['ids'], e['mask'].view(torch.bool), e['risk'], e['stats']

    def static_bytes(self):
        """Device bytes held by the entries' buffers."""
        total = 0
        for e in self.entries.values():
            for v in e.values():
                if torch.is_tensor(v):
                    total += v.numel() * v.element_size()
            total += e['ws'].bytes()
        return total
