"""CPU restatement of the page summaries the current chunk recomputes each
denoise step: a seeded 4-way k-means of each page's 64 keys and the
reference's summary contract built on the clusters.

TEST INFRASTRUCTURE ONLY (see oracle/reference.py): only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` may import it.

The reference builds the 4 token groups of a page with learned softmax
pooling (local_experiments/review_v1/ops.py:43-59); this path's inputs use
k-means clusters as the groups instead, and everything derived from the groups
follows ops.py:60-75 (RV = local_experiments/review_v1):
  reps    pk_r = bf16(km_r - mean_r km + mean_t k)              (RV/ops.py:60)
  mean    mu   = bf16(mean_t v)                                 (RV/ops.py:61)
  detail  bf16(sum_r HAAR[a,r] (vm_r . bf16(basis)) / 4)        (RV/ops.py:62-64)
  stats   group key variance by 16-dim blocks, |km - pk|, |vm - recon|, V
          spread, |mean v - mu|, max token |v|                  (RV/ops.py:66-75)
"""
from __future__ import annotations

import torch

from .reference import HAAR


def deployed(x):
    return x.to(torch.bfloat16).float()


def kmeans(k, init, iters=4):
    """Lloyd iterations on k [B,64,D] fp32 from initial token indices init
    [B,4]: assign to the nearest centroid (squared distance, ties -> lower
    cluster), then move each non-empty centroid to its cluster mean.  Returns
    (centroids [B,4,D], last assignment [B,64], smallest relative gap between
    the best and second-best distance of any token in any iteration [B])."""
    b, t, d = k.shape
    cent = k.gather(1, init.long()[..., None].expand(-1, -1, d)).clone()
    assign = None
    margin = torch.full((b,), torch.inf)
    for _ in range(iters):
        dist = ((k[:, :, None, :] - cent[:, None, :, :]) ** 2).sum(-1)          # [B,64,4]
        top2 = dist.topk(2, dim=-1, largest=False).values
        gap = (top2[..., 1] - top2[..., 0]) / top2[..., 1].clamp_min(1e-30)
        margin = torch.minimum(margin, gap.amin(-1))
        assign = dist.argmin(-1)
        for r in range(4):
            member = (assign == r).float()
            cnt = member.sum(1)
            mean = (member[..., None] * k).sum(1) / cnt.clamp_min(1)[:, None]
            cent[:, r] = torch.where(cnt[:, None] > 0, mean, cent[:, r])
    return cent, assign, margin


def summaries(k, v, basis, init, iters=4):
    """k, v [H,P,64,D] (bf16 values), basis [H,D,8], init [H,P,4] -> dict of
    keys [H,P,4,D], mean [H,P,D], detail [H,P,3,8], stats [H,P,4,12] (bf16)
    and margin [H,P] (k-means near-tie gap)."""
    h, p, t, d = k.shape
    kb = k.float().reshape(h * p, t, d)
    vb = v.float().reshape(h * p, t, d)
    cent, assign, margin = kmeans(kb, init.reshape(h * p, 4), iters)
    onehot = torch.stack([(assign == r).float() for r in range(4)], -1)        # [B,64,4]
    cnt = onehot.sum(1)                                                         # [B,4]
    vmean = vb.mean(1)
    vm = torch.where(cnt[..., None] > 0, torch.einsum('btr,btd->brd', onehot, vb) / cnt.clamp_min(1)[..., None],
                     vmean[:, None, :])
    pk = deployed(cent - cent.mean(1, keepdim=True) + kb.mean(1, keepdim=True))
    mu = deployed(vmean)
    bas = deployed(basis).repeat_interleave(p, 0)                               # [B,D,8]
    code = vm @ bas                                                             # [B,4,8]
    ha = torch.tensor(HAAR, dtype=torch.float32)
    detail = deployed(torch.einsum('ar,brk->bak', ha, code) / 4)
    recon = mu[:, None, :] + torch.einsum('ar,bak,bdk->brd', ha, detail, bas)
    stats = torch.zeros(h * p, 4, 12)
    for r in range(4):
        w = onehot[..., r]
        var = (w[..., None] * (kb - cent[:, r:r + 1]) ** 2).sum(1) / cnt[:, r].clamp_min(1)[:, None]
        stats[:, r, :8] = var.reshape(-1, 8, 16).mean(-1)
        spread = (w * ((vb - vm[:, r:r + 1]) ** 2).sum(-1)).sum(1) / cnt[:, r].clamp_min(1)
        stats[:, r, 10] = spread.sqrt()
    stats[..., 8] = (cent - pk).norm(dim=-1)
    stats[..., 9] = (vm - recon).norm(dim=-1)
    stats[:, 0, 11] = (vmean - mu).norm(dim=-1)
    stats[:, 1, 11] = vb.norm(dim=-1).amax(1)
    bf = lambda x, *shape: x.reshape(h, p, *shape).to(torch.bfloat16)
    return dict(keys=bf(pk, 4, d), mean=bf(mu, d), detail=bf(detail, 3, 8), stats=bf(stats, 4, 12),
                margin=margin.reshape(h, p))
