"""Seeded synthetic inputs for the page-sparse attention call.

Shapes follow the streaming Wan-1.3B runtime the path serves: 12 heads of
128 dims, 3 latent frames of 1536 tokens per chunk (4608 queries, 72 query
blocks of 64), and a window of F frames = 24*F pages of 64 tokens.

Everything here runs on the CPU with a ``torch.Generator`` so the HIP path and
the oracle see identical bytes.  Summaries are the reference's tensor contract
(``Summary(keys[H,P,4,D], mean[H,P,D], detail[H,P,3,8], stats[H,P,4,12])``,
local_experiments/review_v1/ops.py:30-37,66-75) built from a seeded 4-way
k-means of each page's keys instead of the reference's learned pooling; the
basis is the per-head top-8 right singular vectors of page-centred V.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from .ops import HAAR, Summary

SEED_BASE = 0x55A0_0000
TOKENS_PER_FRAME = 1536
PAGES_PER_FRAME = 24
GRID_H, GRID_W = 32, 48
HEADS, HEAD_DIM = 12, 128
QUERY_FRAMES = 3
CURRENT_PAGES = 72
ANCHOR_PAGES = 24
# 16 evenly spaced probe rows of each 64-query block:
# torch.linspace(0,63,16).round() (local_experiments/video_runtime_v1/runtime.py:84).
PROBE_OFFSETS = (0, 4, 8, 13, 17, 21, 25, 29, 34, 38, 42, 46, 50, 55, 59, 63)


def seed_for(cfg: int, layer: int = 0, step: int = 0, tensor_id: int = 0) -> int:
    return SEED_BASE + 1_000_000 * cfg + 1_000 * layer + 10 * step + tensor_id


def rope_params(max_len: int, dim: int, theta: float = 10000.0) -> torch.Tensor:
    """Complex rotary table, as wan/modules/model.py:29-36."""
    freqs = torch.outer(torch.arange(max_len, dtype=torch.float64),
                        1.0 / torch.pow(theta, torch.arange(0, dim, 2, dtype=torch.float64) / dim))
    return torch.polar(torch.ones_like(freqs), freqs)


def rope_table(head_dim: int = HEAD_DIM, max_len: int = 1024) -> torch.Tensor:
    """[max_len, head_dim/2] complex128: 22 temporal, 21 h, 21 w pairs for d=128
    (wan/modules/causal_model.py:500-505)."""
    d = head_dim
    return torch.cat([rope_params(max_len, d - 4 * (d // 6)),
                      rope_params(max_len, 2 * (d // 6)),
                      rope_params(max_len, 2 * (d // 6))], dim=1)


def apply_rope(x: torch.Tensor, first_frame: int, freqs: torch.Tensor) -> torch.Tensor:
    """x [L, H, D] (L a multiple of 1536) rotated at frame first_frame + i // 1536,
    (h, w) = divmod(i % 1536, 48); follows causal_rope_apply
    (wan/modules/causal_model.py:27-55). Returns float64."""
    L, H, D = x.shape
    c = D // 2
    ct, ch = c - 2 * (c // 3), c // 3
    frames = L // TOKENS_PER_FRAME
    ft, fh, fw = freqs.split([ct, ch, ch], dim=1)
    f = torch.cat([
        ft[first_frame:first_frame + frames].view(frames, 1, 1, -1).expand(frames, GRID_H, GRID_W, -1),
        fh[:GRID_H].view(1, GRID_H, 1, -1).expand(frames, GRID_H, GRID_W, -1),
        fw[:GRID_W].view(1, 1, GRID_W, -1).expand(frames, GRID_H, GRID_W, -1),
    ], dim=-1).reshape(L, 1, c)
    z = torch.view_as_complex(x.to(torch.float64).reshape(L, H, c, 2).contiguous())
    return torch.view_as_real(z * f).reshape(L, H, D)


def haar(dtype=torch.float32) -> torch.Tensor:
    return torch.tensor(HAAR, dtype=dtype)


def pca_basis(v_pages: torch.Tensor, rank: int = 8) -> torch.Tensor:
    """Per-head top-`rank` right singular vectors of page-centred V.
    v_pages [H, P, 64, D] -> basis [H, D, rank] float32, sign fixed so the
    largest-magnitude component of each vector is positive."""
    H, P, T, D = v_pages.shape
    x = (v_pages.double() - v_pages.double().mean(2, keepdim=True)).reshape(H, P * T, D)
    cov = x.transpose(1, 2) @ x
    _, vec = torch.linalg.eigh(cov)            # ascending eigenvalues
    basis = vec[..., -rank:].flip(-1)           # [H, D, rank], descending
    idx = basis.abs().argmax(1, keepdim=True)
    sign = torch.sign(basis.gather(1, idx))
    sign[sign == 0] = 1
    return (basis * sign).float()


def kmeans_init(heads: int, pages: int, generator: torch.Generator) -> torch.Tensor:
    """Seeded distinct initial tokens [H, P, 4] (int64) of each page's 4-way
    k-means."""
    return torch.rand(heads * pages, 64, generator=generator).argsort(-1)[:, :4].reshape(heads, pages, 4)


def kmeans_summaries(k: torch.Tensor, v: torch.Tensor, basis: torch.Tensor,
                     generator, iters: int = 4) -> Summary:
    """Page summaries from a seeded 4-way k-means of each page's 64 keys.

    k, v: [H, P, 64, D] (bf16-rounded values); basis [H, D, 8]; generator: a
    torch.Generator for kmeans_init, or the [H, P, 4] initial tokens.
    Reps are the cluster key means re-centred so their mean equals the page key
    mean (local_experiments/review_v1/ops.py:60); detail is the Haar contrast of
    cluster V means projected on the bf16 basis (ops.py:63-64); stats use each
    cluster as the token group (ops.py:68-75).
    """
    H, P, T, D = k.shape
    kf = k.float()
    vf = v.float()
    B = H * P
    kb = kf.reshape(B, T, D)
    vb = vf.reshape(B, T, D)
    # seeded distinct initial tokens per page
    init = (generator if isinstance(generator, torch.Tensor) else kmeans_init(H, P, generator)).reshape(B, 4)
    cent = kb.gather(1, init[..., None].expand(-1, -1, D)).clone()
    assign = None
    for _ in range(iters):
        dist = torch.stack([(kb - cent[:, r:r + 1]).square().sum(-1) for r in range(4)], -1)  # [B,64,4]
        assign = dist.argmin(-1)                                             # ties -> lowest cluster
        onehot = torch.nn.functional.one_hot(assign, 4).float()              # [B,64,4]
        cnt = onehot.sum(1)                                                  # [B,4]
        sums = onehot.transpose(1, 2) @ kb                                   # [B,4,D]
        upd = sums / cnt.clamp_min(1)[..., None]
        cent = torch.where(cnt[..., None] > 0, upd, cent)
    onehot = torch.nn.functional.one_hot(assign, 4).float()
    cnt = onehot.sum(1)
    occupied = cnt > 0
    km = cent                                                              # cluster key means
    vmean_page = vb.mean(1)                                                # [B,D]
    vm = torch.where(occupied[..., None], (onehot.transpose(1, 2) @ vb) / cnt.clamp_min(1)[..., None],
                     vmean_page[:, None, :])                               # cluster V means
    deployed = lambda x: x.to(torch.bfloat16).float()
    pk = deployed(km - km.mean(1, keepdim=True) + kb.mean(1, keepdim=True))
    mu = deployed(vmean_page)
    bas = deployed(basis).reshape(H, 1, D, 8).expand(H, P, D, 8).reshape(B, D, 8)
    code = vm @ bas                                                        # [B,4,8]
    ha = haar()
    detail = deployed(torch.einsum('ar,brk->bak', ha, code) / 4)
    recon = mu[:, None, :] + torch.einsum('ar,bak,bdk->brd', ha, detail, bas)
    stats = torch.zeros(B, 4, 12)
    var = torch.stack([((kb - km[:, r:r + 1]).square() * onehot[..., r:r + 1]).sum(1)
                       for r in range(4)], 1) / cnt.clamp_min(1)[..., None]     # [B,4,D]
    stats[..., :8] = var.reshape(B, 4, 8, 16).mean(-1)
    stats[..., 8] = (km - pk).norm(dim=-1)
    stats[..., 9] = (vm - recon).norm(dim=-1)
    vdev = torch.stack([((vb - vm[:, r:r + 1]).square().sum(-1) * onehot[..., r]).sum(1)
                        for r in range(4)], 1)
    stats[..., 10] = (vdev / cnt.clamp_min(1)).sqrt()
    stats[:, 0, 11] = (vmean_page - mu).norm(dim=-1)
    stats[:, 1, 11] = vb.norm(dim=-1).amax(1)
    return Summary(pk.reshape(H, P, 4, D).to(torch.bfloat16).contiguous(),
                   mu.reshape(H, P, D).to(torch.bfloat16).contiguous(),
                   detail.reshape(H, P, 3, 8).to(torch.bfloat16).contiguous(),
                   stats.reshape(H, P, 4, 12).to(torch.bfloat16).contiguous())


@dataclass
class CallInputs:
    """One sparse-attention call: q [1,N,H,D], k/v [1,64P,H,D] bf16 (the
    resident-cache layout), summaries over the P window pages, basis [H,D,8],
    theta [H,4] and the own page of each query block."""
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    summary: Summary
    basis: torch.Tensor
    theta: torch.Tensor
    own: torch.Tensor
    pages: int

    def to(self, device) -> "CallInputs":
        return CallInputs(self.q.to(device), self.k.to(device), self.v.to(device),
                          Summary(*(getattr(self.summary, n).to(device) for n in Summary.FIELDS)),
                          self.basis.to(device), self.theta.to(device), self.own.to(device), self.pages)


def make_call(cfg: int, frames: int, layer: int = 1, step: int = 0, heads: int = HEADS,
              query_frames: int = QUERY_FRAMES, rope: bool = True) -> CallInputs:
    """Seeded inputs for one call with a window of `frames` latent frames.

    Q/K/V ~ N(0,1), RoPE at window-local positions (queries are the last
    `query_frames` frames), rounded to bf16."""
    D = HEAD_DIM
    L = frames * TOKENS_PER_FRAME
    N = query_frames * TOKENS_PER_FRAME
    P = frames * PAGES_PER_FRAME
    g = torch.Generator().manual_seed(seed_for(cfg, layer, step, 0))
    q = torch.randn(N, heads, D, generator=g)
    k = torch.randn(L, heads, D, generator=g)
    v = torch.randn(L, heads, D, generator=g)
    if rope:
        freqs = rope_table(D)
        q = apply_rope(q, frames - query_frames, freqs)
        k = apply_rope(k, 0, freqs)
    q = q.to(torch.bfloat16)
    k = k.to(torch.bfloat16)
    v = v.to(torch.bfloat16)
    kp = k.transpose(0, 1).reshape(heads, P, 64, D)
    vp = v.transpose(0, 1).reshape(heads, P, 64, D)
    basis = pca_basis(vp.float())
    gs = torch.Generator().manual_seed(seed_for(cfg, layer, step, 1))
    summary = kmeans_summaries(kp, vp, basis, gs)
    theta = torch.tensor([1.0, 1.0, 1.0, 0.5]).expand(heads, 4).contiguous()
    T = N // 64
    own = (torch.arange(T) + P - T)[None].expand(heads, -1).contiguous()
    return CallInputs(q[None].contiguous(), k[None].contiguous(), v[None].contiguous(), summary,
                      basis, theta, own, P)


def quota_table(cfg: int, layers: int = 29, steps: int = 4, heads: int = HEADS,
                mean_total: float = 40.8, a_range=(4, 36), b_range=(0, 40), window: int = 0) -> torch.Tensor:
    """Seeded per-(step, layer, head) (A, B) exact-page quotas with A+B
    constant over the heads of each (step, layer) and averaging `mean_total`;
    `window` seeds one table per window position (chunk) of a stream, as the
    reference's table has one per window.  Returns int64 [steps, layers,
    heads, 2]."""
    g = torch.Generator().manual_seed(seed_for(cfg, window, 0, 7))
    lo_n = a_range[0] + b_range[0]
    hi_n = a_range[1] + b_range[1]
    out = torch.empty(steps, layers, heads, 2, dtype=torch.int64)
    base = int(math.floor(mean_total))
    frac = mean_total - base
    for s in range(steps):
        for l in range(layers):
            n = base + int(torch.rand(1, generator=g).item() < frac)
            jitter = int(torch.randint(-4, 5, (1,), generator=g).item())
            n = max(lo_n, min(hi_n, n + jitter))
            a_lo = max(a_range[0], n - b_range[1])
            a_hi = min(a_range[1], n - b_range[0])
            a = torch.randint(a_lo, a_hi + 1, (heads,), generator=g)
            out[s, l, :, 0] = a
            out[s, l, :, 1] = n - a
    return out


def reader_weights(cfg: int = 3, hidden: int = 256) -> dict:
    """Seeded Full_Pset model weights, fp32 N(0, 0.02), in torch's [out, in]
    Linear layout.  Structure of the reference models:
    LocalReader.page = Linear(712,hidden) -> GELU -> Linear(hidden,85)
    (local_experiments/e27_adaptive_query/coefficients.py:4-8,
    local_experiments/e29_local_reader/core.py:6-10); AdaptivePhi.page =
    Linear(712,hidden) -> GELU -> Linear(hidden,32) and AdaptivePhi.query =
    Linear(128,8,bias=False) (local_experiments/e27_adaptive_query/core.py:8-11);
    the reader projection B [128,16] (fp64 at use) is N(0,1)/sqrt(128)."""
    g = torch.Generator().manual_seed(seed_for(cfg, 0, 0, 5))

    def normal(*shape, std=0.02):
        return (torch.randn(*shape, generator=g) * std).contiguous()

    return dict(
        reader_w1=normal(hidden, 712), reader_b1=normal(hidden),
        reader_w2=normal(85, hidden), reader_b2=normal(85),
        phi_w1=normal(hidden, 712), phi_b1=normal(hidden),
        phi_w2=normal(32, hidden), phi_b2=normal(32),
        wq=normal(8, HEAD_DIM),
        B=(torch.randn(HEAD_DIM, 16, generator=g, dtype=torch.float64) / math.sqrt(HEAD_DIM)).contiguous(),
    )
