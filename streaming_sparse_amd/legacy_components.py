"""Attention dispatcher with the reference's signatures, on the HIP library.

Mirrors local_experiments/video_runtime_v1/legacy_components.py:
``attention(q,k,v,s,basis,ids,workspace,*,bf16_av=True)`` (:24-46) and
``risk(probes,z,summary,theta)`` (:14-22).  Every call goes to libssattn.so;
there is no CPU or eager-torch fallback.
"""
from __future__ import annotations

import math

import torch

from . import _lib
from .ops import Summary

HEAD_DIM = 128


_SUMMARY_INNER = (('keys', (4, HEAD_DIM)), ('mean', (HEAD_DIM,)), ('detail', (3, 8)), ('stats', (4, 12)))


def _check_summary(s: Summary, h: int, p: int):
    """Head-page capacity of the summary slab after checking that each field
    is a bf16 [H, >=p, ...] page slice of a contiguous [H, Pcap, ...] slab
    (shape and stride arithmetic only: no tensor views are built)."""
    hp = s.head_pages
    for name, inner in _SUMMARY_INNER:
        t = getattr(s, name)
        if t.dtype != torch.bfloat16:
            raise TypeError(f"summary.{name} must be bf16")
        shape, stride = t.shape, t.stride()
        if shape[0] != h or shape[1] < p:
            raise ValueError(f"summary.{name} shape {tuple(shape)} does not cover {h} heads x {p} pages")
        want = [1] * len(inner)
        for i in range(len(inner) - 2, -1, -1):
            want[i] = want[i + 1] * inner[i + 1]
        n = want[0] * inner[0]
        if tuple(shape[2:]) != inner or list(stride[2:]) != want or stride[1] != n or stride[0] != hp * n:
            raise ValueError(f"summary.{name} must be a page slice of a contiguous [H,{hp},...] slab")
    return hp


def kv_strides(k: torch.Tensor, v: torch.Tensor):
    """(token stride, head stride) in elements of the resident K/V cache.
    Token-major contiguous [1,L,H,D] or the head-major strided variant
    (legacy_components.py:28-30)."""
    d = k.shape[-1]
    major = k.stride(1) == d and k.stride(2) >= k.shape[1] * d
    if k.is_contiguous() and v.is_contiguous():
        return k.stride(1), k.stride(2)
    if major and k.stride() == v.stride():
        return k.stride(1), k.stride(2)
    raise ValueError("k/v must be contiguous [1,L,H,D] or head-major with equal strides")


REP_OP_ELEMS = 512
"""bf16 elements of one detail operand tile (16 pages, 1024 bytes)."""


def rep_tiles(pages: int) -> int:
    """Operand tiles a window of `pages` pages needs: ceil(pages / 16)."""
    return (pages + 15) // 16


def check_rep_ops(t: torch.Tensor, h: int, pages: int, name: str = "rep_ops"):
    if t.dtype != torch.bfloat16 or not t.is_contiguous() or t.dim() != 3 or t.shape[0] != h or \
            t.shape[1] < rep_tiles(pages) or t.shape[2] != REP_OP_ELEMS:
        raise ValueError(f"{name} must be a contiguous bf16 [H,>={rep_tiles(pages)},{REP_OP_ELEMS}] tensor")


@torch.no_grad()
def rep_operands(s: Summary, pages: int, out: torch.Tensor):
    """The compensation's detail operand tiles [H,>=ceil(P/16),512] (bf16) of
    the summary's detail rows, in the order the fused kernel reads them."""
    h = s.mean.shape[0]
    hp = _check_summary(s, h, pages)
    check_rep_ops(out, h, pages, "out")
    _lib.check(_lib.lib().ssa_rep_operands(_lib.ptr(s.detail), _lib.ptr(out), h, pages, hp, out.shape[1],
                                           _lib.stream_handle(out.device)), "ssa_rep_operands")
    return out


SINGLE_AV = False
"""Module switch of the P.V arithmetic, as the reference's (legacy_components.py:4):
False (default) runs the reference's two-term bf16 product (hi + lo parts of
each probability, HIGH_PRECISION_AV=not SINGLE_AV at legacy_components.py:49;
the tail's _av at tuned_attention.py:16-18); True runs one bf16 product."""


_WORKSPACE_BYTES = {}


@torch.no_grad()
def split_workspace(workspace, n_tokens, heads, pages, count, flags, device):
    """The attention call's workspace from `workspace`, or None when the call
    needs none: the tiles past the last multiple of the device's CU count
    run as pieces whose states a second kernel merges, and a staged call
    (flags bit 2) keeps two states per tile.  The size is asked of the
    library once per (shape, flags, device)."""
    key = (n_tokens, heads, pages, count, flags, device)
    need = _WORKSPACE_BYTES.get(key)
    if need is None:
        need = _lib.lib().ssa_attention_workspace_bytes(n_tokens, heads, pages, count, flags)
        if need < 0:
            raise RuntimeError("ssa_attention_workspace_bytes failed")
        _WORKSPACE_BYTES[key] = need
    return workspace.tensor('ssa_split', (need,), device, torch.uint8) if need > 0 else None


def attention(q, k, v, s, basis, ids, workspace, *, bf16_av=True, single_av=None, all_pages=False,
              rep_ops=None, split=True, staged=False):
    """Exact attention over the LUT pages + summary compensation + merge.

    q [1,N,H,128] bf16 contiguous; k, v [1,64P,H,128] bf16 (resident cache);
    s a Summary covering the P pages; basis [H,128,8]; ids [H,N/64,C] int32 with
    own page first (entries outside [0,P), the -1 padding of a shorter table,
    are not read).  Returns ``out`` [1,N,H,128] bf16, owned by `workspace`
    and overwritten by the next call.

    Arithmetic: every probability multiplies V as the two-term bf16 product
    hi + lo, the reference's exact stage; the compensation weighs the page
    means and the Haar contrasts of the detail rows with two-term (hi + lo)
    bf16 weights, as the reference's ``bf16_av=True`` tail does
    (tuned_attention.py:16-18,60-62), and applies the rank-8 code to the
    bf16 basis as a two-term bf16 product (the reference: tf32x3,
    tuned_attention.py:71).  ``bf16_av=False`` (the reference's tf32x3 tail)
    maps to the same two-term products, the closest this kernel runs.
    ``single_av=True`` (default: the module's SINGLE_AV) opts into one bf16
    term for every probability and weight.  ``all_pages=True`` states that every row
    of ids lists each page exactly once (a dense call): two query blocks then
    share each K/V page load and ids are not read.  ``rep_ops``: the
    [H,>=ceil(P/16),512] detail operand tiles of `s` when the caller already
    has them (route(..., rep_out=...) writes them on the side); otherwise
    they are computed here.  ``split=False`` runs every tile in one piece
    (no split workspace; the tiles past the last multiple of the CU count
    otherwise run as two pieces each).  ``staged=True`` runs the exact pages
    and the compensation as two launches whose states a merge kernel
    combines (the reference's exact kernel + tail + merge), so a profiler
    shows the two stages apart; not with ``all_pages``."""
    _, n, h, d = q.shape
    p = k.shape[1] // 64
    count = ids.shape[-1]
    if d != HEAD_DIM or q.dtype != torch.bfloat16 or not q.is_contiguous():
        raise ValueError("q must be contiguous [1,N,H,128] bf16")
    if k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16 or k.shape != v.shape:
        raise ValueError("k, v must be bf16 with equal shapes")
    tok, head = kv_strides(k, v)
    hp = _check_summary(s, h, p)
    if ids.dtype != torch.int32 or ids.shape[:2] != (h, n // 64):
        raise ValueError("ids must be int32 [H,N/64,C]")
    ids = ids.contiguous()

    def buf(name, shape, dtype):
        return workspace.tensor('ssa_' + name, shape, q.device, dtype)

    if all_pages and count != p:
        raise ValueError("all_pages needs a table of exactly P pages per row")
    b = basis if (basis.dtype == torch.bfloat16 and basis.is_contiguous()) else basis.to(torch.bfloat16).contiguous()
    if b.shape != (h, HEAD_DIM, 8):
        raise ValueError("basis must be [H,128,8]")
    if all_pages and (n // 64) % 2 == 0:
        # the two-block dense kernel reads no operand tiles
        ops, ntiles = None, 0
    elif rep_ops is not None:
        check_rep_ops(rep_ops, h, p)
        ops, ntiles = rep_ops, rep_ops.shape[1]
    else:
        ops = rep_operands(s, p, buf('rep_ops', (h, rep_tiles(p), REP_OP_ELEMS), torch.bfloat16))
        ntiles = ops.shape[1]
    out = buf('out', q.shape, q.dtype)
    single = SINGLE_AV if single_av is None else bool(single_av)
    if staged and all_pages:
        raise ValueError("a staged call is a general call (not all_pages)")
    flags = (0 if single else 1) | (2 if all_pages else 0) | (4 if staged else 0)
    split = split_workspace(workspace, n, h, p, count, flags, q.device) if (split or staged) else None
    _lib.check(_lib.lib().ssa_attention(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(s.keys), _lib.ptr(s.mean),
                                        _lib.ptr(b), _lib.ptr(ops), _lib.ptr(ids), _lib.ptr(out), n, h, p, hp, ntiles,
                                        count, tok, head, flags, _lib.ptr(split),
                                        0 if split is None else split.numel(), _lib.stream_handle(q.device)),
               "ssa_attention")
    return out


@torch.no_grad()
def risk(probes, z, summary, theta, *, z_tol=1e-4):
    """Per-page risk [H,T,P] fp32 from probe rows [H,T,16,128].

    The kernel forms the probe logits on chip from `probes` and the rep keys.
    `z` is the reference's precomputed logits bf16(probe).bf16(repK)^T/sqrt(D)
    [H,T,16,P,4] (legacy_components.py:14-22 consumes them); a z that is not
    those of `probes` (beyond fp32 summation order: |dz| <= z_tol (1 + |z|))
    is rejected with ValueError rather than silently ignored.  z=None skips
    the check."""
    h, t, m, d = probes.shape
    p = summary.mean.shape[1]
    if m != 16 or d != HEAD_DIM:
        raise ValueError("probes must be [H,T,16,128]")
    hp = _check_summary(summary, h, p)
    if z is not None:
        if tuple(z.shape) != (h, t, m, p, 4):
            raise ValueError(f"z must be [H,T,16,P,4] = {(h, t, m, p, 4)}, got {tuple(z.shape)}")
        pf = probes.to(torch.bfloat16).float().reshape(h, t * m, d)
        kf = summary.keys.float().reshape(h, p * 4, d)
        mine = torch.bmm(pf, kf.transpose(1, 2).contiguous()).reshape(h, t, m, p, 4) / math.sqrt(d)
        zf = z.float()
        if not bool(((mine - zf).abs() <= z_tol * (1 + zf.abs())).all()):
            raise ValueError("z is not the probe logits of `probes` and the summary's rep keys")
    pr = probes.to(torch.bfloat16).contiguous()
    th = theta.float().contiguous()
    out = torch.empty(h, t, p, device=probes.device, dtype=torch.float32)
    _lib.check(_lib.lib().ssa_route(_lib.ptr(pr), t * m * d, m * d, d, 1, _lib.ptr(summary.keys),
                                    _lib.ptr(summary.stats), _lib.ptr(th), None, None, _lib.ptr(out), None, None,
                                    None, h, t, p, hp, 0, -1, 0, None, None, 0, 0.0, None, None,
                                    _lib.stream_handle(probes.device)), "ssa_route")
    return out
