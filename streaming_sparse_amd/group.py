"""Clean-commit token grouping on the HIP library: the order in which a
committed chunk's 4608 tokens fill its 72 pages.

Mirrors GroupingOps.group (local_experiments/review_v1/runtime.py:57-68): the
grouping features of SparseLayer.group_features
(local_experiments/all_sparse_model.py:16-23), the balanced splits of
local_experiments/response_hard.py:20-31 (3,3,2,2,2 over the chunk, then 2,2
inside each page), Config.page_order (local_experiments/review_v1/ops.py:25-28)
and, for the first chunk, the stable re-sort by frame of
local_experiments/video_runtime_v1/runtime.py:358-363.  Layers are grouped in
one batch, as the reference's batched clean commit does
(local_experiments/video_runtime_v1/runtime.py:330-354).  Nothing here
computes on the CPU.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib, workload

CHUNK_TOKENS = 4608
FEATURES = 32
PAGES = 72


@dataclass
class GroupWeights:
    """Per-layer grouping parameters (the reference's learned bank, group_v and
    group_gate): bank [L,H,32,128], group_v [L,H,128,32], gate [L,H,32] fp32."""
    bank: torch.Tensor
    group_v: torch.Tensor
    gate: torch.Tensor

    @staticmethod
    def seeded(layers, heads, seed, device):
        """Synthetic weights with the reference's initial structure
        (all_sparse_model.py:9-11): group_v = the row-normalised bank,
        transposed; gate near 0.1."""
        g = torch.Generator().manual_seed(workload.seed_for(seed, 0, 0, 11))
        bank = torch.randn(layers, heads, FEATURES, 128, generator=g)
        gv = torch.nn.functional.normalize(bank, dim=-1).transpose(-1, -2).contiguous()
        gate = 0.1 + 0.05 * torch.randn(layers, heads, FEATURES, generator=g)
        f32 = dict(device=device, dtype=torch.float32)
        return GroupWeights(bank.to(**f32).contiguous(), gv.to(**f32).contiguous(), gate.to(**f32).contiguous())


def page_destinations(history_pages: int, current_pages: int = PAGES):
    """Destination page of each grouped page under Config.page_order
    (RV/ops.py:25-28): the `drop` early pages go first.  None = identity."""
    drop = (current_pages - history_pages % current_pages) % current_pages
    if not drop:
        return None
    early = [i * current_pages // drop for i in range(drop)]
    order = early + [i for i in range(current_pages) if i not in early]
    dst = [0] * current_pages
    for q, pg in enumerate(order):
        dst[pg] = q
    return torch.tensor(dst, dtype=torch.int32)


@torch.no_grad()
def order(k, v, weights: GroupWeights, *, first_chunk=False, page_dst=None, workspace=None, out=None):
    """k, v: the chunk's tokens of L layers, [L, 4608, H, 128] bf16 (or
    [4608, H, 128] for one layer), token-major; weights for those layers;
    page_dst: page_destinations(...) (CPU int32 [72]) or None.  Returns order
    [L, H, 4608] int32 (chunk token of each destination position, head by
    head)."""
    if k.dim() == 3:
        k, v = k[None], v[None]
    L, n, h, d = k.shape
    if n != CHUNK_TOKENS or d != 128 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16 or \
            k.shape != v.shape or k.stride() != v.stride() or k.stride(-1) != 1:
        raise ValueError("k, v must be bf16 [L, 4608, H, 128] with equal strides")
    for name, t, shape in (('bank', weights.bank, (L, h, FEATURES, 128)), ('group_v', weights.group_v,
                                                                              (L, h, 128, FEATURES)),
                           ('gate', weights.gate, (L, h, FEATURES))):
        if tuple(t.shape) != shape or t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError(f"weights.{name} must be contiguous fp32 {shape}")
    dev = k.device
    b = L * h

    def buf(name, shape, dtype):
        if workspace is None:
            return torch.empty(shape, device=dev, dtype=dtype)
        return workspace.tensor('group_' + name, shape, dev, dtype)

    sx = buf('x', (2, b, CHUNK_TOKENS, FEATURES), torch.float64)
    si = buf('ids', (2, b, CHUNK_TOKENS), torch.int32)
    res = out if out is not None else buf('order', (L, h, CHUNK_TOKENS), torch.int32)
    pd = None
    if page_dst is not None:
        pd = page_dst.to(device=dev, dtype=torch.int32).contiguous()
        if pd.shape != (PAGES,) or sorted(page_dst.tolist()) != list(range(PAGES)):
            raise ValueError("page_dst must be a permutation of the 72 pages")
    _lib.check(_lib.lib().ssa_group_order(_lib.ptr(k), _lib.ptr(v), k.stride(0), k.stride(1), k.stride(2),
                                          _lib.ptr(weights.bank), _lib.ptr(weights.group_v), _lib.ptr(weights.gate),
                                          _lib.ptr(pd), int(bool(first_chunk)), L, h, _lib.ptr(sx), _lib.ptr(si),
                                          _lib.ptr(res), _lib.stream_handle(dev)), "ssa_group_order")
    return res
