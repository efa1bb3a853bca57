"""CPU restatement of the reference's clean-commit token grouping.

TEST INFRASTRUCTURE ONLY, like oracle/reference.py: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` may import it.

Path aliases: RV = local_experiments/review_v1, LE = local_experiments,
VR = local_experiments/video_runtime_v1.

A committed chunk's 4608 tokens are reordered into 72 pages of 64 before the
pages are summarised (RV/runtime.py:57-68 GroupingOps.group):
  features   f = key + 0.1 tanh(gate) response        (LE/all_sparse_model.py:16-23)
  balanced   recursive splits of 3,3,2,2,2 by a power-iteration direction,
             stable sorts                              (LE/response_hard.py:20-31)
  inner      the same with splits 2,2 inside each page of 64
  pages      Config.page_order                         (RV/ops.py:25-28)
  chunk 0    tokens stably re-sorted by frame so the anchor frame fills pages
             0..23                                     (VR/runtime.py:358-363)
The reference runs these in float32; this restatement runs them in float64
(the library's kernels do too), so the two orders agree except where two
scores fall within float32 rounding of each other.
"""
from __future__ import annotations

import math

import torch

SPLITS = (3, 3, 2, 2, 2)
INNER = (2, 2)
CHUNK_TOKENS = 4608
PAGE = 64


def group_features(k, v, bank, group_v, gate):
    """SparseLayer.group_features (LE/all_sparse_model.py:16-23) for one chunk
    per head: k, v [H, T, D] (bf16 values), bank [H, R, D], group_v [H, D, R],
    gate [H, R] -> f [H, T, R] float64."""
    k = k.double()
    v = v.double()
    kc = k - k.mean(-2, keepdim=True)
    score = torch.einsum('htd,hrd->htr', kc, bank.double()) / math.sqrt(k.shape[-1])
    rms = score.square().mean((-2, -1), keepdim=True).sqrt().clamp_min(1e-6)
    key = score / rms
    a = score.softmax(-2)
    vp = torch.einsum('htd,hdr->htr', v, group_v.double())
    mean = (a * vp).sum(-2, keepdim=True)
    response = a * k.shape[-2] * (vp - mean)
    response = response / response.square().mean((-2, -1), keepdim=True).sqrt().clamp_min(1e-6)
    return key + 0.1 * gate.double().tanh()[:, None, :] * response


def balanced(x, factors, iterations=4):
    """balanced (LE/response_hard.py:20-31): x [H, n, d] -> ids [H, n]; at each
    level every group is centred, a direction starts at the one-hot of its
    highest-variance dimension, takes `iterations` power steps (normalised,
    norm clamped at 1e-8), and the group is stably sorted by the projection;
    the sorted group is split into `factor` equal parts for the next level."""
    h, n, d = x.shape
    ids = torch.arange(n).expand(h, n).clone()
    groups = 1
    for factor in factors:
        size = n // groups
        x = x.reshape(h * groups, size, d)
        ids = ids.reshape(h * groups, size)
        xc = x - x.mean(1, keepdim=True)
        var = xc.square().mean(1)
        direction = torch.zeros_like(var).scatter_(1, var.argmax(-1, keepdim=True), 1.0)
        for _ in range(iterations):
            direction = torch.bmm(xc.transpose(1, 2), torch.bmm(xc, direction.unsqueeze(-1))).squeeze(-1)
            direction = direction / direction.norm(dim=-1, keepdim=True).clamp_min(1e-8)
        order = torch.bmm(xc, direction.unsqueeze(-1)).squeeze(-1).argsort(dim=-1, stable=True)
        x = x.gather(1, order[:, :, None].expand_as(x))
        ids = ids.gather(1, order)
        groups *= factor
    return ids.reshape(h, n)


def page_order(history_pages, current_pages=72):
    """Config.page_order (RV/ops.py:25-28): the `drop` early pages first."""
    drop = (current_pages - history_pages % current_pages) % current_pages
    early = [i * current_pages // drop for i in range(drop)] if drop else []
    return torch.tensor(early + [i for i in range(current_pages) if i not in early])


def group_order(k, v, bank, group_v, gate, pages=None, first_chunk=False):
    """The token order of GroupingOps.group (RV/runtime.py:60-68): k, v
    [H, 4608, D] -> order [H, 4608] (destination position -> chunk token); with
    `first_chunk`, the stable re-sort by frame of VR/runtime.py:358-363."""
    h, n, _ = k.shape
    f = group_features(k, v, bank, group_v, gate)
    order = balanced(f, SPLITS)
    fp = f.gather(1, order[:, :, None].expand_as(f))
    inner = balanced(fp.reshape(-1, PAGE, f.shape[-1]), INNER).reshape(h, n // PAGE, PAGE)
    pages = torch.arange(n // PAGE) if pages is None else pages
    order = order.reshape(h, n // PAGE, PAGE).gather(2, inner)[:, pages].flatten(1)
    if first_chunk:
        perm = torch.argsort(order // 1536, dim=1, stable=True)
        order = order.gather(1, perm)
    return order
