"""Full_Pset swap correction on the HIP library: reader weights, page
encodings and the correction step of the router.

Mirrors local_experiments/video_runtime_v1/page.py (``encode``/``read``),
VideoRuntime.encode (local_experiments/video_runtime_v1/runtime.py:160-164)
and the ``full_pset`` branch of BatchGraphs.compute
(reproduction/vbench_current/graph.py:169-208).  Every step runs in
libssattn.so; nothing here computes on the CPU.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib
from .ops import Summary

HEAD_DIM = 128
COEF_STRIDE = 128      # bf16 per page: co[85] | 0 x 11 | A[32]
COEF_A = 96
CAND = 48
CAND_VALS = 34
ROW_VALS = 52
ROW_SPLIT = 2          # page ranges per pair of query blocks in the rows kernel
POOL_INTS = 64


class Reader:
    """Frozen LocalReader + AdaptivePhi + projection B on one device, in the
    kernels' layout.  ``weights`` holds torch-layout fp32 tensors
    (reader_w1/b1/w2/b2, phi_w1/b1/w2/b2, wq [8,128], B [128,16])."""

    def __init__(self, weights: dict, device):
        dev = torch.device(device)
        f32 = dict(device=dev, dtype=torch.float32)
        self.hidden = int(weights['reader_w1'].shape[0])
        if weights['phi_w1'].shape[0] != self.hidden or not 0 < self.hidden <= 256:
            raise ValueError("reader and phi hidden widths must match and be <= 256")
        self.w1t = torch.cat([weights['reader_w1'], weights['phi_w1']], 0).t().contiguous().to(**f32)
        self.b1 = torch.cat([weights['reader_b1'], weights['phi_b1']]).contiguous().to(**f32)
        self.w2r = weights['reader_w2'].contiguous().to(**f32)
        self.b2r = weights['reader_b2'].contiguous().to(**f32)
        self.w2p = weights['phi_w2'].contiguous().to(**f32)
        self.b2p = weights['phi_b2'].contiguous().to(**f32)
        self.wq = weights['wq'].contiguous().to(**f32)
        self.B = weights['B'].to(device=dev, dtype=torch.float64).contiguous()


@dataclass
class Encoding:
    """Per-page encodings over a slab of `pages` capacity: coef [H,Pe,128] bf16
    (co [5,17] at 0..84, A [8,4] at 96..127), mean [H,Pe,16] and detail
    [H,Pe,3,16] fp64 (the reference's en['co'/'A'/'mean'/'detail'])."""
    coef: torch.Tensor
    mean: torch.Tensor
    detail: torch.Tensor

    @staticmethod
    def empty(heads, pages, device):
        return Encoding(torch.zeros(heads, pages, COEF_STRIDE, device=device, dtype=torch.bfloat16),
                        torch.zeros(heads, pages, 16, device=device, dtype=torch.float64),
                        torch.zeros(heads, pages, 3, 16, device=device, dtype=torch.float64))

    @property
    def co(self):
        return self.coef[..., :85].unflatten(-1, (5, 17))

    @property
    def A(self):
        return self.coef[..., COEF_A:].unflatten(-1, (8, 4))


def _summary_ok(s: Summary):
    hp = s.head_pages
    for name, t, inner in (('keys', s.keys, 512), ('mean', s.mean, 128), ('detail', s.detail, 24),
                           ('stats', s.stats, 48)):
        if t.dtype != torch.bfloat16 or t.stride(0) != hp * inner or not t[0].is_contiguous():
            raise ValueError(f"summary.{name} must be a page slice of a contiguous bf16 slab")
    return hp


@torch.no_grad()
def encode(summary: Summary, basis: torch.Tensor, reader: Reader, out: Encoding | None = None,
           first: int = 0, pages: int | None = None) -> Encoding:
    """Encode pages [first, first + pages) of `summary` (a slab or a prefix
    slice) into `out` (allocated over the summary's pages when None)."""
    h = summary.mean.shape[0]
    hp = _summary_ok(summary)
    pages = summary.mean.shape[1] - first if pages is None else pages
    dev = summary.mean.device
    if out is None:
        out = Encoding.empty(h, summary.mean.shape[1], dev)
    b = basis if (basis.dtype == torch.bfloat16 and basis.is_contiguous()) else basis.to(torch.bfloat16).contiguous()
    if b.shape != (h, HEAD_DIM, 8):
        raise ValueError("basis must be [H,128,8]")
    ep = out.coef.shape[1]
    _lib.check(_lib.lib().ssa_encode(
        _lib.ptr(summary.keys), _lib.ptr(summary.mean), _lib.ptr(summary.detail), _lib.ptr(summary.stats), hp,
        _lib.ptr(b), _lib.ptr(reader.w1t), _lib.ptr(reader.b1), _lib.ptr(reader.w2r), _lib.ptr(reader.b2r),
        _lib.ptr(reader.w2p), _lib.ptr(reader.b2p), _lib.ptr(reader.B), _lib.ptr(out.coef), _lib.ptr(out.mean),
        _lib.ptr(out.detail), ep, h, first, pages, reader.hidden, _lib.stream_handle(dev)), "ssa_encode")
    return out


@torch.no_grad()
def encode_layers(summaries, bases, reader: Reader, outs, first: int, pages: int):
    """encode() of the same page range over several layers in one launch
    (ssa_encode_layers): one summary slab, basis and encoding per layer (at
    most 32), with equal slab and encoding capacities; the reader weights are
    shared.  Equal to an encode() per layer, bit for bit."""
    n = len(summaries)
    if not 1 <= n <= 32 or not len(bases) == len(outs) == n:
        raise ValueError("one slab, basis and encoding per layer, 1..32 layers")
    h = summaries[0].mean.shape[0]
    hp = _summary_ok(summaries[0])
    ep = outs[0].coef.shape[1]
    dev = summaries[0].mean.device
    bs = []
    for s_, basis, out in zip(summaries, bases, outs):
        if _summary_ok(s_) != hp or s_.mean.shape[0] != h or s_.mean.device != dev:
            raise ValueError("every layer's slab must have the first one's heads and capacity")
        if out.coef.shape != (h, ep, COEF_STRIDE) or not out.coef.is_contiguous() or \
                out.mean.shape != (h, ep, 16) or not out.mean.is_contiguous() or \
                out.detail.shape != (h, ep, 3, 16) or not out.detail.is_contiguous():
            raise ValueError("every layer's encoding must have the first one's shape, contiguous")
        b = basis if (basis.dtype == torch.bfloat16 and basis.is_contiguous()) else \
            basis.to(torch.bfloat16).contiguous()
        if b.shape != (h, HEAD_DIM, 8):
            raise ValueError("basis must be [H,128,8]")
        bs.append(b)
    _lib.check(_lib.lib().ssa_encode_layers(
        n, _lib.ptrs([s_.keys for s_ in summaries]), _lib.ptrs([s_.mean for s_ in summaries]),
        _lib.ptrs([s_.detail for s_ in summaries]), _lib.ptrs([s_.stats for s_ in summaries]), hp, _lib.ptrs(bs),
        _lib.ptr(reader.w1t), _lib.ptr(reader.b1), _lib.ptr(reader.w2r), _lib.ptr(reader.b2r), _lib.ptr(reader.w2p),
        _lib.ptr(reader.b2p), _lib.ptr(reader.B), _lib.ptrs([o.coef for o in outs]), _lib.ptrs([o.mean for o in outs]),
        _lib.ptrs([o.detail for o in outs]), ep, h, first, pages, reader.hidden, _lib.stream_handle(dev)),
        "ssa_encode_layers")
    return outs


@torch.no_grad()
def correct(q, summary: Summary, encoding: Encoding, reader: Reader, risk, lse, mask, ids, own, heads,
            workspace=None, want_scores=False, no_alloc=False, probe_layout=None):
    """Full_Pset correction of the scoped `heads` in place on `mask` (uint8 or
    bool storage, [H,T,P]) and `ids` [H,T,C] from the intersection router,
    whose `risk` and per-probe `lse` ([H,T,16], route(..., lse_out=...)) it
    reads.  q [1,N,H,128] bf16 (probe rows at the reference offsets).
    no_alloc: run ssa_pset_noalloc, whose scratch is the library's own
    device array (at most 216 scoped (head, block) rows; concurrent calls on
    one device race), instead of workspace scratch.
    probe_layout: (head, block, row strides in elements, gathered) of a q in
    another layout, e.g. the reference's [H, T, n, D] blocks (gathered = 1:
    q holds the 16 probe rows of each block); default: q is [1,N,H,128].
    Returns (stats int64 [3] = executed, rows, non-finite scores; per-row
    dict)."""
    h, t, p = risk.shape
    d = HEAD_DIM
    dev = q.device
    if probe_layout is None:
        if q.dim() != 4 or q.shape[2] != h or q.shape[1] != 64 * t:
            raise ValueError("q must be [1,N,H,128] (or pass probe_layout)")
        probe_layout = (d, 64 * h * d, h * d, 0)
    if torch.is_tensor(heads) and heads.device == dev and heads.dtype == torch.int32 and heads.dim() == 1:
        # a device list the caller has checked (distinct ids in [0, H)): read by the kernels as it is
        # at launch, so a captured graph follows the caller's updates
        hs = heads
        if hs.numel() == 0:
            raise ValueError("full_pset heads must not be empty")
    else:
        head_list = [int(i) for i in heads]
        if not head_list or len(set(head_list)) != len(head_list) or min(head_list) < 0 or max(head_list) >= h:
            raise ValueError(f"full_pset heads must be distinct ids in [0,{h})")
        key = ('pset_heads', tuple(head_list), torch.device(dev), torch.int32)
        if workspace is not None and key in workspace.entries:
            hs = workspace.entries[key]
        else:
            hs = torch.tensor(head_list, dtype=torch.int32).to(dev)
            if workspace is not None:
                workspace.entries[key] = hs
    n = hs.numel()
    hp = _summary_ok(summary)
    if encoding.coef.shape[1] < p:
        raise ValueError("encoding does not cover the window")
    if lse is None or lse.shape != (h, t, 16) or lse.dtype != torch.float32 or not lse.is_contiguous():
        raise ValueError("lse must be the router's contiguous [H,T,16] float32 probe log-sum-exp")

    def buf(name, shape, dtype):
        if workspace is None:
            return torch.empty(shape, device=dev, dtype=dtype)
        return workspace.tensor('pset_' + name, shape, dev, dtype)

    gain = buf('gain', (n, t), torch.float64)
    info = buf('info', (n, t, 3), torch.int32)
    scores = buf('scores', (n, t, 16, 32), torch.float64) if want_scores else None
    stats = buf('stats', (3,), torch.int64)
    mask_u8 = mask.view(torch.uint8) if mask.dtype == torch.bool else mask
    ow = None if own is None else own.to(device=dev, dtype=torch.int32).contiguous()
    head = (_lib.ptr(q), *probe_layout, _lib.ptr(summary.keys), hp, _lib.ptr(encoding.coef),
            _lib.ptr(encoding.mean), _lib.ptr(encoding.detail), encoding.coef.shape[1], _lib.ptr(reader.wq),
            _lib.ptr(risk), _lib.ptr(lse), _lib.ptr(mask_u8), _lib.ptr(ids), _lib.ptr(ow), _lib.ptr(hs), n)
    tail = (_lib.ptr(gain), _lib.ptr(info), _lib.ptr(scores), _lib.ptr(stats), h, t, p, ids.shape[-1],
            _lib.stream_handle(dev))
    pool = None
    if no_alloc:
        _lib.check(_lib.lib().ssa_pset_noalloc(*head, *tail), "ssa_pset_noalloc")
    else:
        cand = buf('cand', (n, t, 16, CAND, CAND_VALS), torch.float64)
        rows = buf('rows', (n, t, 16, ROW_SPLIT, ROW_VALS), torch.float64)
        pool = buf('pool', (n, t, POOL_INTS), torch.int32)
        _lib.check(_lib.lib().ssa_pset(*head, _lib.ptr(cand), _lib.ptr(rows), _lib.ptr(pool), *tail), "ssa_pset")
    return stats, dict(gain=gain, executed=info[..., 0], argmax=info[..., 1], nonfinite=info[..., 2],
                       scores=scores, pool=pool)
