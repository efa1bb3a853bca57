"""CPU restatement of the reference's Full_Pset swap correction (stage 2).

TEST INFRASTRUCTURE ONLY, like oracle/reference.py: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` may import it.

Path aliases: VR = local_experiments/video_runtime_v1, VB =
reproduction/vbench_current, LE = local_experiments.

Pipeline for the scoped heads of one call (VB/graph.py:169-210):
  encodings  co, A, meanB, detailB        (VR/page.py:6-14, VR/runtime.py:89,160-164)
  readout    rp[16], beta per probe/page  (VR/page.py:17-21)
  log mass   lm = LSE_r z - LSE_{p,r} z   (VB/graph.py:181)
  center     approx - sum_p e^lm approx   (VB/graph.py:199-201)
  pools      8 removes + 16 adds per partition, same-partition legality;
             a 72-page window: 8 current removes x the top 16 adds
                                          (VB/quota_pool.py:3-46)
  scores     FP64 proxy gain per (remove, add), mean over probes
                                          (VR/scores.py:54-91)
  apply      argmax; execute iff gain > 0 and all finite (VR/scores.py:102-107)
  LUT        own first, then descending risk over the new mask (VB/graph.py:210)
"""
from __future__ import annotations

import math

import torch

from .reference import HAAR, ANCHORS, CURRENT

FEATURES = 712


# ---------------------------------------------------------------- encoding --

def page_features(keys, mean, detail, stats):
    """[H,P,712] fp32: each of keys(512), mean(128), detail(24), stats(48)
    divided by (its RMS + 1e-4) (VR/page.py:8-9; LE/e27_adaptive_query/core.py:4-6)."""
    parts = [keys.float().flatten(2), mean.float(), detail.float().flatten(2), stats.float().flatten(2)]
    return torch.cat([x / (x.square().mean(-1, keepdim=True).sqrt() + 1e-4) for x in parts], -1)


def mlp(f, w1, b1, w2, b2):
    """Linear -> exact (erf) GELU -> Linear in fp32 (LE/e27_adaptive_query/core.py:10,
    LE/e27_adaptive_query/coefficients.py:6); weights in torch [out, in] layout."""
    h = torch.nn.functional.linear(f, w1, b1)
    h = torch.nn.functional.gelu(h)
    return torch.nn.functional.linear(h, w2, b2)


def encode(keys, mean, detail, stats, basis, w):
    """Page encodings (VR/page.py:6-14 with coeff_bf16, VR/runtime.py:160-164):
    co [H,P,5,17] bf16 (reader), A [H,P,8,4] bf16 (phi), meanB = mean.B
    [H,P,16] fp64, detailB = detail.(bf16(basis)^T B) [H,P,3,16] fp64."""
    h, p = mean.shape[:2]
    f = page_features(keys, mean, detail, stats)
    co = mlp(f, w['reader_w1'], w['reader_b1'], w['reader_w2'], w['reader_b2']).reshape(h, p, 5, 17).bfloat16()
    a = mlp(f, w['phi_w1'], w['phi_b1'], w['phi_w2'], w['phi_b2']).reshape(h, p, 8, 4).bfloat16()
    b = w['B'].double()
    mean_b = mean.double() @ b
    projected = basis.bfloat16().double().transpose(1, 2) @ b                  # [H,8,16] (VR/runtime.py:89)
    detail_b = torch.matmul(detail.double(), projected[:, None])               # [H,P,3,16]
    return dict(co=co, A=a, mean=mean_b, detail=detail_b)


# ----------------------------------------------------------------- readout --

def read(probes, co, a, wq):
    """Reader readout (VR/page.py:17-21): u = phi.query(probe) [8];
    F_j = tanh(sum_i u_i A_pij); val = co_p0 + sum_j F_j co_p(j+1).
    Returns rp [H,T,M,P,16] and beta [H,T,M,P] (fp32)."""
    u = probes.float() @ wq.float().t()
    f = torch.tanh(torch.einsum('htmi,hpij->htmpj', u, a.float()))
    val = co.float()[:, None, None, :, 0] + torch.einsum('htmpj,hpjk->htmpk', f, co.float()[:, :, 1:])
    return val[..., :16], val[..., 16]


def log_mass(z):
    """Per probe, normalised page log mass in fp64 (VB/graph.py:176-181):
    lm = LSE_r z - LSE_{p,r} z.  z [H,T,M,P,4]."""
    lz = z.double().logsumexp(-1)
    return lz - lz.logsumexp(-1, keepdim=True)


def center(z, lm, mean_b, detail_b):
    """Summary readout in the B-projected space, centred on its mass-weighted
    mean (VB/graph.py:199-201): approx = meanB + sum_a c_a detailB_a with the
    Haar contrasts c of the softmax over the page's 4 reps."""
    ha = torch.tensor(HAAR, dtype=torch.float64)
    contrast = torch.einsum('htmpr,ar->htmpa', z.double().softmax(-1), ha)
    approx = mean_b[:, None, None] + torch.einsum('htmpa,hpak->htmpk', contrast, detail_b)
    return approx - (lm.exp()[..., None] * approx).sum(-2, keepdim=True)


# ------------------------------------------------------------------- pools --

def stratified_pool(risk, mask, own):
    """Per partition (history [24,P-72), current [P-72,P)): the 8 lowest-risk
    movable selected pages (removes) and the 16 highest-risk unselected pages
    (adds), stable order; legal = movable remove x unselected add, same
    partition (VB/quota_pool.py:3-15)."""
    p = risk.shape[-1]
    page = torch.arange(p)
    movable = mask & (page >= ANCHORS) & (page != own[..., None])
    removes, adds = [], []
    for lo, hi in ((ANCHORS, p - CURRENT), (p - CURRENT, p)):
        score = risk[..., lo:hi]
        removes.append(score.masked_fill(~movable[..., lo:hi], torch.inf).argsort(dim=-1, stable=True)[..., :8] + lo)
        adds.append(score.masked_fill(mask[..., lo:hi], -torch.inf).argsort(dim=-1, descending=True, stable=True)[..., :16] + lo)
    r, a = torch.cat(removes, -1), torch.cat(adds, -1)
    legal = movable.gather(-1, r)[..., :, None] & ~mask.gather(-1, a)[..., None, :]
    legal = legal & ((r[..., :, None] >= p - CURRENT) == (a[..., None, :] >= p - CURRENT))
    return r, a, legal


def first_chunk_pool(risk, mask, own):
    """Pool of a 72-page window, where the anchor frame is the chunk's first
    frame and every non-anchor page is current (VB/quota_pool.py:21-33).
    Removes: the movable pages (selected, not an anchor, not own) by
    ascending risk, at most 8, then the anchor pages other than own in page
    order.  Adds: the unselected pages by descending risk, then the selected
    pages in page order, 32 slots.  Legal: the movable removes x the first
    16 add slots (whatever those hold).  Ties -> lower page."""
    p = risk.shape[-1]
    page = torch.arange(p)
    movable = mask & (page >= ANCHORS) & (page != own[..., None])
    by_risk = risk.masked_fill(~movable, torch.inf).sort(dim=-1, stable=True).indices
    n_mov = movable.sum(-1, keepdim=True).clamp_max(8)
    # anchor pages other than own, ascending (own, if an anchor, goes last)
    stand_in = torch.where((page < ANCHORS) & (page != own[..., None]), page, p + page).sort(dim=-1).values
    slot = torch.arange(16)
    pad = stand_in.gather(-1, (slot - n_mov).clamp_min(0))
    remove = torch.where(slot < n_mov, by_risk[..., :16], pad)
    add = risk.masked_fill(mask, -torch.inf).sort(dim=-1, descending=True, stable=True).indices[..., :32]
    legal = (slot < n_mov)[..., None] & (torch.arange(32) < 16)
    return remove, add, legal


def pool(risk, mask, own):
    """Stratified pool with slot padding (VB/quota_pool.py:32-46): invalid
    remove slot i -> anchor page i; invalid add slot j -> the j-th smallest page
    that is neither selected nor a valid add.  Padded slots are never legal.
    When fewer than j + 1 such pages exist, slot j holds P, as the
    reference's `spare` does (`topk` of a tensor filled with P): page P is
    past the window, and grouped_scores reads it as an empty candidate (zero
    mass, zero values).  A 72-page window takes the first chunk's pool
    (first_chunk_pool)."""
    if risk.shape[-1] == CURRENT:
        return first_chunk_pool(risk, mask, own)
    r, a, legal = stratified_pool(risk, mask, own)
    valid_remove = mask.gather(-1, r) & (r != own[..., None])
    anchor = torch.arange(r.size(-1))
    r = torch.where(valid_remove, r, anchor)
    used = mask.scatter(-1, a, True)
    pages = torch.arange(mask.size(-1))
    spare = torch.where(used, mask.size(-1), pages).topk(a.size(-1), largest=False).values
    a = torch.where(mask.gather(-1, a), spare, a)
    return r, a, legal


# ------------------------------------------------------------------ scores --

def _gather(x, ids):
    index = ids[:, None].expand(-1, x.shape[1], -1)
    if x.ndim == 4:
        index = index[..., None].expand(-1, -1, -1, x.shape[-1])
    return x.gather(2, index)


def _exclude(logs, values):
    """Leave-one-out log mass and mixture of a candidate group
    (VR/scores.py:34-47)."""
    k = logs.shape[-1]
    eye = torch.eye(k, dtype=torch.bool)
    excluded = logs[:, :, None, :].expand(-1, -1, k, -1).masked_fill(eye, -torch.inf)
    lse = excluded.logsumexp(-1)
    # a group whose other members all have zero mass has no mixture (its
    # weight e^(lse - den) is 0); zero instead of softmax's 0/0
    mix = torch.where(torch.isfinite(lse)[..., None], excluded.softmax(-1) @ values, 0.0)
    return lse, mix


def grouped_scores(rp, beta, lm, cen, mask, remove, add):
    """FP64 proxy gain of every (remove, add) swap (VR/scores.py:54-91).
    rp [B,M,P,16], beta/lm [B,M,P], cen [B,M,P,16], mask [B,P], remove [B,R],
    add [B,A] -> [B,R,A] = mean over probes of 2 E.delta - |delta|^2, where
    E = target - H and delta is the change of the mixture H after the swap."""
    rp, beta, lm, cen = (x.double() for x in (rp, beta, lm, cen))
    p = mask.shape[-1]
    if bool((add >= p).any()):
        # an add slot past the spare pages holds page P (pool): one more page
        # of zero mass and zero values, outside the selection
        def pad(x, value):
            return torch.cat([x, torch.full_like(x[:, :, :1], value)], 2)
        rp, cen, beta, lm = pad(rp, 0.0), pad(cen, 0.0), pad(beta, 0.0), pad(lm, -torch.inf)
        mask = torch.cat([mask, torch.zeros_like(mask[:, :1])], 1)
    le = lm + beta
    v = cen + rp
    logs = torch.where(mask[:, None], le, lm)
    cur = cen + mask[:, None, :, None] * rp
    H = (logs.softmax(-1)[..., None] * cur).sum(2)
    target = (le.softmax(-1)[..., None] * v).sum(2)
    E = target - H
    candidates = torch.zeros_like(mask).scatter(1, remove, True).scatter(1, add, True)
    bg = logs.masked_fill(candidates[:, None], -torch.inf)
    lb = bg.logsumexp(-1)
    ob = (bg.softmax(-1)[..., None] * cur).sum(2)
    lr, er, cr, pr = _gather(lm, remove), _gather(le, remove), _gather(cen, remove), _gather(rp, remove)
    la, ea, ca, pa = _gather(lm, add), _gather(le, add), _gather(cen, add), _gather(rp, add)
    rx, ro = _exclude(er, cr + pr)
    ax, ao = _exclude(la, ca)
    den = torch.logaddexp(lb[:, :, None, None], rx[:, :, :, None])
    den = torch.logaddexp(den, ax[:, :, None, :])
    den = torch.logaddexp(den, lr[:, :, :, None])
    den = torch.logaddexp(den, ea[:, :, None, :])
    new = (lb[:, :, None, None] - den).exp()[..., None] * ob[:, :, None, None]
    new = new + (rx[:, :, :, None] - den).exp()[..., None] * ro[:, :, :, None]
    new = new + (ax[:, :, None, :] - den).exp()[..., None] * ao[:, :, None]
    new = new + (lr[:, :, :, None] - den).exp()[..., None] * cr[:, :, :, None]
    new = new + (ea[:, :, None, :] - den).exp()[..., None] * (ca + pa)[:, :, None]

    def endpoint(l, e, c, p_, ids, axis):
        bb = _gather(beta, ids)
        if axis == 'r':
            l, e, c, p_, bb = l[:, :, :, None], e[:, :, :, None], c[:, :, :, None], p_[:, :, :, None], bb[:, :, :, None]
        else:
            l, e, c, p_, bb = l[:, :, None, :], e[:, :, None, :], c[:, :, None], p_[:, :, None], bb[:, :, None, :]
        exact = (e - den).exp()
        approx = (l - den).exp()
        diff = torch.where(bb.abs() < .5, approx * torch.expm1(bb.clamp(-.5, .5)), exact - approx)
        return diff[..., None] * (c - H[:, :, None, None]) + exact[..., None] * p_

    delta = endpoint(la, ea, ca, pa, add, 'a') - endpoint(lr, er, cr, pr, remove, 'r')
    bad = (logs.amax(-1)[:, :, None, None] - den > 80) | (~torch.isfinite(delta).all(-1))
    delta = torch.where(bad[..., None], new - H[:, :, None, None], delta)
    return (2 * (E[:, :, None, None] * delta).sum(-1) - delta.square().sum(-1)).mean(1)


def apply_best(mask, remove, add, scores):
    """Execute the best swap iff its gain > 0 and every score is finite
    (VR/scores.py:102-107).  Returns (mask, gain, executed, flat argmax)."""
    flat = scores.flatten(1)
    gain, j = flat.max(-1)
    execute = (gain > 0) & torch.isfinite(flat).all(-1)
    rr = remove.gather(1, (j // add.shape[-1])[:, None])
    aa = add.gather(1, (j % add.shape[-1])[:, None])
    # rows that execute swap rr out and aa in; the others keep their mask
    # (their argmax may name an illegal slot: a selected page or page P)
    p = mask.shape[-1]
    swapped = torch.cat([mask, torch.zeros_like(mask[:, :1])], 1)
    swapped = swapped.scatter(1, rr, False).scatter(1, aa, True)[:, :p]
    result = torch.where(execute[:, None], swapped, mask)
    return result, gain, execute, j


# ---------------------------------------------------------------- pipeline --

def correct(probes, z, risk, mask, own, enc, wq, heads):
    """Full_Pset correction of the scoped heads (VB/graph.py:169-208).

    probes [H,T,16,D] (bf16 values), z [H,T,16,P,4] probe logits, risk [H,T,P],
    mask [H,T,P] bool selection, own [H,T], enc = encode(...) over all P pages,
    wq [8,D] phi.query weight, heads list of scoped head ids.  Returns the full
    new mask plus per-row (scores [Hs,T,R,A] with illegal pairs at -1e30,
    gain, executed, argmax, remove, add, legal) and the reference's stats
    (executed count, rows, non-finite scores)."""
    h, t, m, p, _ = z.shape
    hs = torch.as_tensor(heads, dtype=torch.long)
    zs, pr, rk, mk, ow = z[hs], probes[hs], risk[hs], mask[hs], own[hs]
    en = {k: v[hs] for k, v in enc.items()}
    lm = log_mass(zs)
    r, a, legal = pool(rk, mk, ow)
    rp, beta = read(pr, en['co'], en['A'], wq)
    cen = center(zs, lm, en['mean'], en['detail'])
    b = hs.numel() * t
    scores = grouped_scores(rp.reshape(b, m, p, 16), beta.reshape(b, m, p), lm.reshape(b, m, p),
                            cen.reshape(b, m, p, 16), mk.reshape(b, p), r.reshape(b, -1), a.reshape(b, -1))
    scores = scores.masked_fill(~legal.reshape_as(scores), -1e30)
    new, gain, executed, j = apply_best(mk.reshape(b, p), r.reshape(b, -1), a.reshape(b, -1), scores)
    full = mask.clone()
    full[hs] = new.reshape(hs.numel(), t, p)
    stats = torch.stack((executed.sum(), torch.tensor(b), (~torch.isfinite(scores)).sum()))
    rows = dict(scores=scores.reshape(hs.numel(), t, 16, 32), gain=gain.reshape(hs.numel(), t),
                executed=executed.reshape(hs.numel(), t), argmax=j.reshape(hs.numel(), t),
                remove=r, add=a, legal=legal, lm=lm, rp=rp, beta=beta, center=cen)
    return full, rows, stats
