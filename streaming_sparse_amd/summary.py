"""Current-chunk page summaries on the HIP library (4-iteration k-means reps,
V mean, Haar/rank-8 detail, routing stats), written into a summary slab.

The reference recomputes the current chunk's summaries on every denoise
input (local_experiments/video_runtime_v1/runtime.py:213-227, fused kernels in
local_experiments/video_runtime_v1/summary_moments.py:113-137) and writes them
into its [H, Pcap, ...] slabs; ``build`` does the same for pages
[first, first + pages) of the resident K/V cache.  Nothing here computes on
the CPU.
"""
from __future__ import annotations

import torch

from . import _lib
from .legacy_components import HEAD_DIM, kv_strides
from .ops import Summary


# field -> (inner shape, page / inner strides) of a contiguous [H, Pcap, ...] bf16 slab
_SLAB = (('keys', (4, 128), (512, 128, 1)), ('mean', (128,), (128, 1)), ('detail', (3, 8), (24, 8, 1)),
         ('stats', (4, 12), (48, 12, 1)))


def _check_slab(out: Summary, h: int, first: int, pages: int) -> int:
    hp = out.head_pages
    for name, shape, strides in _SLAB:
        t = getattr(out, name)
        if t.dtype != torch.bfloat16 or t.stride() != (hp * strides[0],) + strides or t.shape[0] != h or \
                t.shape[2:] != shape:
            raise ValueError(f"out.{name} must be a page slice of a contiguous bf16 [H,Pcap,...] slab")
        if first + pages > t.shape[1]:
            raise ValueError(f"out.{name} does not cover pages [{first}, {first + pages})")
    return hp


def _check_init(init, h: int, pages: int):
    ini = init if (init.dtype == torch.int32 and init.is_contiguous()) else init.to(torch.int32).contiguous()
    if ini.shape != (h, pages, 4):
        raise ValueError("init must be [H, pages, 4]")
    return ini


def _bf16_basis(basis):
    return basis if (basis.dtype == torch.bfloat16 and basis.is_contiguous()) else basis.to(torch.bfloat16).contiguous()


def _check_cache(k, v, first: int, pages: int):
    _, L, h, d = k.shape
    if d != HEAD_DIM or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16 or k.shape != v.shape:
        raise ValueError("k, v must be bf16 [1, 64P, H, 128]")
    if first < 0 or pages <= 0 or (first + pages) * 64 > L:
        raise ValueError("page range outside the K/V window")
    return h


@torch.no_grad()
def build(k, v, basis, init, out: Summary, first: int, pages: int, iters: int = 4, src=None) -> Summary:
    """k, v [1, 64P, H, 128] bf16 cache; basis [H,128,8]; init [H, pages, 4]
    initial k-means tokens (0..63) per page; out: a summary slab (or prefix
    slice) whose pages [first, first + pages) are overwritten.

    src = (src_k, src_v), each [64 pages, H, 128] bf16 with unit head-dim
    stride: those rows are first written into the cache pages [first, first
    + pages) (the window write of VR/runtime.py:205-206) in the same pass
    that summarises them (ssa_summary_write); cache and summaries equal a
    copy followed by the summary, bit for bit."""
    h = _check_cache(k, v, first, pages)
    d = HEAD_DIM
    if src is not None:
        sk, sv = src
        if sk.shape != (64 * pages, h, d) or sv.shape != sk.shape or sk.dtype != torch.bfloat16 or \
                sv.dtype != torch.bfloat16 or sk.stride() != sv.stride() or sk.stride(2) != 1 or \
                sk.device != k.device or sv.device != k.device:
            raise ValueError("src must be two bf16 [64*pages, H, 128] tensors with equal strides on the cache device")
    hp = _check_slab(out, h, first, pages)
    ini = _check_init(init, h, pages)
    b = _bf16_basis(basis)
    tok, head = kv_strides(k, v)
    if src is not None:
        _lib.check(_lib.lib().ssa_summary_write(_lib.ptr(sk), _lib.ptr(sv), sk.stride(0), sk.stride(1), _lib.ptr(k),
                                                _lib.ptr(v), tok, head, _lib.ptr(ini), _lib.ptr(b), _lib.ptr(out.keys),
                                                _lib.ptr(out.mean), _lib.ptr(out.detail), _lib.ptr(out.stats), hp, h,
                                                first, pages, iters, _lib.stream_handle(k.device)),
                   "ssa_summary_write")
        return out
    _lib.check(_lib.lib().ssa_summary(_lib.ptr(k), _lib.ptr(v), tok, head, _lib.ptr(ini), _lib.ptr(b),
                                      _lib.ptr(out.keys), _lib.ptr(out.mean), _lib.ptr(out.detail),
                                      _lib.ptr(out.stats), hp, h, first, pages, iters,
                                      _lib.stream_handle(k.device)), "ssa_summary")
    return out


@torch.no_grad()
def build_layers(ks, vs, bases, init, outs, first: int, pages: int, iters: int = 4):
    """build() of the same page range over several layers in one launch
    (ssa_summary_layers): ks, vs, bases and outs hold one cache, basis and
    summary slab per layer (at most 32 layers), with equal cache strides and
    slab capacities; init is shared.  Equal to a build() per layer, bit for
    bit."""
    n = len(ks)
    if not 1 <= n <= 32 or not len(vs) == len(bases) == len(outs) == n:
        raise ValueError("one cache, basis and slab per layer, 1..32 layers")
    h = _check_cache(ks[0], vs[0], first, pages)
    tok, head = kv_strides(ks[0], vs[0])
    hp = outs[0].head_pages
    bs = []
    for k, v, basis, out in zip(ks, vs, bases, outs):
        if _check_cache(k, v, first, pages) != h or kv_strides(k, v) != (tok, head) or k.device != ks[0].device:
            raise ValueError("every layer's cache must have the first one's shape and strides")
        if _check_slab(out, h, first, pages) != hp:
            raise ValueError("every layer's slab must have the first one's capacity")
        b = _bf16_basis(basis)
        if b.shape != (h, HEAD_DIM, 8):
            raise ValueError("basis must be [H,128,8]")
        bs.append(b)
    ini = _check_init(init, h, pages)
    _lib.check(_lib.lib().ssa_summary_layers(
        n, _lib.ptrs(ks), _lib.ptrs(vs), tok, head, _lib.ptr(ini), _lib.ptrs(bs), _lib.ptrs([o.keys for o in outs]),
        _lib.ptrs([o.mean for o in outs]), _lib.ptrs([o.detail for o in outs]), _lib.ptrs([o.stats for o in outs]),
        hp, h, first, pages, iters, _lib.stream_handle(ks[0].device)), "ssa_summary_layers")
    return outs
