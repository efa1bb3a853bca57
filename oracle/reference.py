"""CPU restatement of the reference's page-sparse attention path.

TEST INFRASTRUCTURE ONLY.  This module is the parity oracle: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only to check or time against the HIP path.  The product path
(``streaming_sparse_amd``) never imports it and has no CPU fallback.

Every function restates one routine of jurky123/streaming_sparse in plain torch
on the CPU (float32 by default, float64 on request), citing the reference
file:line it follows.  Path aliases: VR = local_experiments/video_runtime_v1,
RV = local_experiments/review_v1, VB = reproduction/vbench_current.
"""
from __future__ import annotations

import math

import torch

HAAR = ((1, 1, -1, -1), (1, -1, 1, -1), (1, -1, -1, 1))            # RV/ops.py:10
PROBE_OFFSETS = (0, 4, 8, 13, 17, 21, 25, 29, 34, 38, 42, 46, 50, 55, 59, 63)
ANCHORS = 24
CURRENT = 72


def haar(dtype=torch.float32):
    return torch.tensor(HAAR, dtype=dtype)


def deployed(x):
    """bf16 rounding of a stored operand (RV/ops.py:41)."""
    return x.to(torch.bfloat16).float()


# ---------------------------------------------------------------- router ----

def probes(q, offsets=PROBE_OFFSETS):
    """q [1,N,H,D] -> probe rows [H,T,16,D] of each 64-query block
    (VR/runtime.py:84 offsets; VR/route_probes.py:6-21 gather)."""
    _, n, h, d = q.shape
    x = q[0].transpose(0, 1).reshape(h, n // 64, 64, d)
    return x[:, :, list(offsets)].contiguous()


def route_logits(pr, keys, dtype=torch.float32):
    """z = bf16(probe) . bf16(repK)^T * D^-1/2 with fp32 accumulation
    (VR/tensor_bmm.py:56-66, kernel :7-30) -> [H,T,16,P,4]."""
    h, t, m, d = pr.shape
    p = keys.shape[1]
    a = deployed(pr).to(dtype).reshape(h, t * m, d)
    b = deployed(keys).to(dtype).reshape(h, p * 4, d)
    z = torch.bmm(a, b.transpose(1, 2)) * (d ** -0.5)
    return z.reshape(h, t, m, p, 4)


def risk(pr, z, stats, theta, dtype=torch.float32):
    """Per-page risk [H,T,P]: the four features of RV/ops.py:80-111 in the
    deployed form risk_from_logits (VR/runtime.py:27-40; the fused kernels
    VR/risk_online.py:24-59 (_risk_tile), :77-86 (risk), row normaliser
    :88-113): prob = exp(z-max)/sum exp(z-max) over the P*4 reps of
    each probe row, u = max(0, sum_g q2_g*st_g), beta = |q|/sqrt(D)*st_8,
    c = st[p,1,11] + max_p st[p,1,11], value = ((t0 x0 + t1 x1) + t2 x2) + t3 x3,
    mean over the 16 probes."""
    h, t, m, d = pr.shape
    q = deployed(pr).to(dtype)
    st = stats.to(dtype)
    z = z.to(dtype)
    flat = z.flatten(-2)
    mx = flat.amax(-1, keepdim=True)
    den = (flat - mx).exp().sum(-1, keepdim=True)
    prob = ((flat - mx).exp() / den).reshape_as(z)                     # [H,T,M,P,4]
    alpha = prob.sum(-1)
    q2 = q.square().reshape(h, t, m, 8, 16).sum(-1) / d
    qn = q.norm(dim=-1) / math.sqrt(d)
    u = torch.einsum('htmg,hprg->htmpr', q2, st[..., :8]).clamp_min(0)
    beta = qn[..., None, None] * st[:, None, None, :, :, 8]
    bp = st[:, :, 1, 11]
    c = (bp + bp.amax(-1, keepdim=True))[:, None, None]
    x0 = alpha * st[:, None, None, :, 0, 11] + ((prob - alpha[..., None] / 4).abs() * st[:, None, None, :, :, 9]).sum(-1)
    x1 = (prob * u.sqrt() * st[:, None, None, :, :, 10]).sum(-1)
    x2 = c * (prob * beta).sum(-1)
    x3 = c * (prob * (u + beta.square())).sum(-1)
    th = theta.to(dtype)[:, None, None, None, :]
    value = ((x0 * th[..., 0] + x1 * th[..., 1]) + x2 * th[..., 2]) + x3 * th[..., 3]
    return value.sum(2) / m


def route_features(q, keys, stats, dtype=torch.float32):
    """RouteOps.features (RV/ops.py:80-111) for all pages valid: q [H,Q,D] ->
    features [H,Q,P,4] and logZ [H,Q]."""
    h, n, d = q.shape
    q = deployed(q).to(dtype)
    k = deployed(keys).to(dtype)
    st = stats.to(dtype)
    z = torch.einsum('hqd,hprd->hqpr', q, k) / math.sqrt(d)
    logz = z.flatten(2).logsumexp(-1)
    prob = (z - logz[:, :, None, None]).exp()
    alpha = prob.sum(-1)
    q2 = q.square().reshape(h, n, 8, 16).sum(-1) / d
    qn = q.norm(dim=-1) / math.sqrt(d)
    u = torch.einsum('hqg,hprg->hqpr', q2, st[..., :8]).clamp_min(0)
    beta = qn[:, :, None, None] * st[:, None, :, :, 8]
    bp = st[:, :, 1, 11]
    c = bp[:, None, :] + bp.amax(-1)[:, None, None]
    x0 = alpha * st[:, None, :, 0, 11] + ((prob - alpha[..., None] / 4).abs() * st[:, None, :, :, 9]).sum(-1)
    x1 = (prob * u.sqrt() * st[:, None, :, :, 10]).sum(-1)
    x2 = c * (prob * beta).sum(-1)
    x3 = c * (prob * (u + beta.square())).sum(-1)
    return torch.stack((x0, x1, x2, x3), -1), logz


def _rank_desc(score, valid):
    """Stable descending order: larger score first, ties -> lower page index.
    Invalid entries last."""
    s = score.masked_fill(~valid, -torch.inf)
    return s.sort(dim=-1, descending=True, stable=True).indices


def select_base(risk_, own, count):
    """Base tier LUT (VR/runtime.py:279-288): [own, 0..23, the count-25
    highest-risk pages excluding own and anchors, by descending risk]."""
    h, t, p = risk_.shape
    page = torch.arange(p)
    valid = (page[None, None] >= ANCHORS) & (page[None, None] != own[..., None])
    order = _rank_desc(risk_, valid)[..., :count - 1 - ANCHORS]
    frame = page[:ANCHORS].expand(h, t, -1)
    return torch.cat((own[..., None], frame, order), -1).int()


def _keep(scores, slots):
    """_keep (VB/quota_mask.py:7-15) over one partition's rows: the top
    `slots` scores, ties -> lower index; slots <= 0 keeps nothing, slots >= the
    partition size keeps all of it.  Returns the kept column indices."""
    if slots <= 0:
        return scores[..., :0].long()
    return scores.sort(dim=-1, descending=True, stable=True).indices[..., :slots]


def quota_mask(risk_, own, current, total):
    """Anchor/history/current partition selection (VB/quota_mask.py:17-39):
    pages < 24 always; history [24, P-72) keeps its top (total - A); current
    [P-72, P) keeps its top A with own forced (+inf, when own is a current
    page); ties -> lower index.  A 72-page window, whose first frame is the
    anchor frame (VB/graph.py:143-148), keeps the anchors and the top `total`
    of pages [24, 72) with own forced; `current` is then not read."""
    h, t, p = risk_.shape
    mask = torch.zeros(h, t, p, dtype=torch.bool)
    mask[..., :ANCHORS] = True
    if p == CURRENT:
        page = torch.arange(p)
        ranked = risk_.masked_fill(page < ANCHORS, -torch.inf).scatter(-1, own.long()[..., None], torch.inf)
        mask.scatter_(-1, _keep(ranked[..., ANCHORS:], int(total)) + ANCHORS, True)
        return mask
    for hh in range(h):
        a = int(current[hh])
        hist = risk_[hh, :, ANCHORS:p - CURRENT]
        mask[hh].scatter_(-1, _keep(hist, int(total) - a) + ANCHORS, True)
        cur = risk_[hh, :, p - CURRENT:].clone()
        rel = own[hh].long() - (p - CURRENT)
        inside = (rel >= 0) & (rel < CURRENT)
        cur[inside, rel[inside]] = torch.inf
        mask[hh].scatter_(-1, _keep(cur, a) + (p - CURRENT), True)
    return mask


def lut(risk_, mask, own, count):
    """Final page LUT (VB/graph.py:210): topk(count) of risk masked to the
    selection with own = +inf -> own first, then descending risk (ties -> lower
    index; torch.topk leaves tie order unspecified).  When the selection plus
    own holds fewer than `count` pages (quotas clamped to their partitions)
    torch.topk would return arbitrary unselected pages in the remaining slots;
    they are -1 here (the padding of RV/ops.py:115-135), parity unpinned at
    that edge."""
    ranked = risk_.masked_fill(~mask, -torch.inf).scatter(-1, own.long()[..., None], torch.inf)
    vals, idx = ranked.sort(dim=-1, descending=True, stable=True)
    idx = idx[..., :count].int()
    return idx.masked_fill(vals[..., :count] == -torch.inf, -1)


def select_topk(risk_, own, count):
    """Fixed-count selection with own forced, no anchors (RouteOps.select with
    threshold None, RV/ops.py:113-138; VR/fixed_page_select.py:8-47)."""
    ranked = risk_.scatter(-1, own[..., None], torch.inf)
    ids = ranked.sort(dim=-1, descending=True, stable=True).indices[..., :count]
    mask = torch.zeros_like(risk_, dtype=torch.bool).scatter(-1, ids, True)
    return ids.int(), mask


def select_counts(scores, own, *, threshold=None, valid=None, density=0.10, max_fraction=0.25,
                  id_capacity=128):
    """RouteOps.select (RV/ops.py:113-138): the pages ranked by score with
    invalid pages at -inf and own at +inf (ties -> lower page); with a
    threshold, count = clamp(#(score > threshold and valid, own forced), 1,
    cap) and overflow the excess over cap = min(id_capacity, ceil(max_fraction
    P)); without, count = min(max(1, floor(P density)), #valid) and no
    overflow.  ids = the top count pages then -1 up to id_capacity; mask the
    selected pages; residual_risk = the sum of the scores of the valid
    unselected pages (float64 here)."""
    h, t, p = scores.shape
    if valid is None:
        valid = torch.ones(h, t, p, dtype=torch.bool)
    valid = valid.expand(h, t, p)
    cap = min(id_capacity, math.ceil(max_fraction * p))
    ranked = scores.double().masked_fill(~valid, -torch.inf).scatter(-1, own[..., None].long(), torch.inf)
    order = ranked.sort(dim=-1, descending=True, stable=True).indices[..., :min(id_capacity, p)]
    if threshold is None:
        count = torch.full((h, t), max(1, math.floor(p * density)), dtype=torch.long)
        count = torch.minimum(count, valid.sum(-1))
        overflow = torch.zeros_like(count)
    else:
        eligible = ((scores > threshold) & valid).scatter(-1, own[..., None].long(), True)
        wanted = eligible.sum(-1)
        overflow = (wanted - cap).clamp_min(0)
        count = wanted.clamp(1, cap)
    active = torch.arange(order.shape[-1]) < count[..., None]
    ids = order.masked_fill(~active, -1)
    if ids.shape[-1] < id_capacity:
        ids = torch.nn.functional.pad(ids, (0, id_capacity - ids.shape[-1]), value=-1)
    mask = torch.zeros(h, t, p, dtype=torch.bool).scatter(-1, order, active)
    residual = scores.double().masked_fill(mask | ~valid, 0).sum(-1)
    return dict(ids=ids.int(), counts=count.int(), mask=mask, overflow=overflow.int(), residual_risk=residual)


def mask_from_ids(ids, pages):
    """Selected-page set of each (head, block) from its LUT
    (RV/tuned_attention.py:37-40; LE high_sparse_runtime.py:12-17); entries
    outside [0, pages) (padding -1) select nothing."""
    h, t, _ = ids.shape
    ok = (ids >= 0) & (ids < pages)
    col = torch.where(ok, ids.long(), torch.full_like(ids.long(), pages))   # invalid -> a spare column
    return torch.zeros(h, t, pages + 1, dtype=torch.bool).scatter(-1, col, True)[..., :pages]


# ------------------------------------------------------------- attention ----

def selected_attention(q, k, v, s, basis, ids, dtype=torch.float32, tiles=None):
    """SelectedAttention.fixed (RV/runtime.py:107-133): exact softmax attention
    over the LUT pages, summary compensation over the unselected pages (rep
    logits, V mean plus Haar/rank-8 detail through the basis), and the log-mass
    merge.  q [1,N,H,D]; k,v [1,64P,H,D]; s a Summary over the P pages; basis
    [H,D,8]; ids [H,T,C].  Returns [1,N,H,D] in `dtype` (callers round to bf16).
    `tiles` optionally restricts the query blocks evaluated."""
    _, n, h, d = q.shape
    p = k.shape[1] // 64
    count = ids.shape[-1]
    query_all = q[0].transpose(0, 1)
    keys = k[0].transpose(0, 1).reshape(h, p * 64, d)
    values = v[0].transpose(0, 1).reshape(h, p * 64, d)
    reps = s.keys[:, :p].reshape(h, p * 4, d).to(dtype)
    means = s.mean[:, :p].to(dtype)
    detail = s.detail[:, :p].to(dtype).flatten(1, 2)
    bas = deployed(basis).to(dtype)
    ha = haar(dtype)
    mask = mask_from_ids(ids, p)
    offsets = torch.arange(64)
    tiles = range(n // 64) if tiles is None else tiles
    out = torch.zeros(h, n, d, dtype=dtype)
    for tile in tiles:
        query = query_all[:, tile * 64:(tile + 1) * 64].to(dtype)
        sel = ids[:, tile, :count].long()
        # LUT entries outside [0, P) (padding -1) are not read (RV/ops.py:115)
        valid = ((sel >= 0) & (sel < p))[:, :, None].expand(-1, -1, 64).flatten(1)
        tokens = (sel.clamp(0, p - 1)[:, :, None] * 64 + offsets).flatten(1)
        index = tokens[:, :, None].expand(-1, -1, d)
        kk = keys.gather(1, index).to(dtype)
        vv = values.gather(1, index).to(dtype)
        z = torch.bmm(query, kk.transpose(1, 2)) / math.sqrt(d)
        z = z.masked_fill(~valid[:, None, :], -torch.inf)
        ze = z.logsumexp(-1)
        exact = torch.bmm(z.softmax(-1), vv)
        exact = torch.where(torch.isfinite(ze)[..., None], exact, torch.zeros_like(exact))   # no valid entry
        zs = torch.bmm(query, reps.transpose(1, 2)).reshape(h, 64, p, 4) / math.sqrt(d)
        zs = zs.masked_fill(mask[:, tile, None, :, None], -torch.inf)
        zt = zs.flatten(2).logsumexp(-1) + math.log(16)
        normalizer = torch.where(torch.isfinite(zt), zt - math.log(16), torch.zeros_like(zt))
        weights = (zs - normalizer[:, :, None, None]).exp()
        mean = torch.bmm(weights.sum(-1), means)
        contrasts = torch.einsum('hqpr,ar->hqpa', weights, ha)
        code = torch.bmm(contrasts.flatten(2), detail)
        tail = mean + torch.bmm(code, bas.transpose(1, 2))
        total = torch.logaddexp(ze, zt)
        out[:, tile * 64:(tile + 1) * 64] = exact * (ze - total).exp()[..., None] + tail * (zt - total).exp()[..., None]
    return out.transpose(0, 1)[None]


def dense_attention(q, k, v, dtype=torch.float32, chunk=512):
    """Full softmax attention over all window tokens: the all-pages-exact case
    (RV/test_ops.py:19-23 compares against scaled_dot_product_attention)."""
    _, n, h, d = q.shape
    qq = q[0].transpose(0, 1).to(dtype)
    kk = k[0].transpose(0, 1).to(dtype)
    vv = v[0].transpose(0, 1).to(dtype)
    out = torch.empty(h, n, d, dtype=dtype)
    for a in range(0, n, chunk):
        z = torch.bmm(qq[:, a:a + chunk], kk.transpose(1, 2)) / math.sqrt(d)
        out[:, a:a + chunk] = torch.bmm(z.softmax(-1), vv)
    return out.transpose(0, 1)[None]


# ---------------------------------------------------------------- stream ----

def shift_temporal(keys, tokens, freqs, offset):
    """Anchor rebase (LE/anchor_rebase.py:8-18 shift_temporal_, applied by
    VB/phase.py:4-25): the first `tokens` rows of keys [1, L, H, D] get their
    temporal RoPE pairs (the first D/2 - 2 (D/2 // 3) complex pairs)
    multiplied by freqs[offset, :pairs] in complex128 and cast back to the
    keys' dtype; the spatial pairs and the other rows stay bitwise equal.
    Returns a new tensor."""
    out = keys.clone()
    if offset == 0 or tokens == 0:
        return out
    pairs = keys.shape[-1] // 2 - 2 * (keys.shape[-1] // 2 // 3)
    part = out[:, :tokens, :, :pairs * 2]
    z = torch.view_as_complex(part.double().reshape(*part.shape[:-1], pairs, 2).contiguous())
    part.copy_(torch.view_as_real(z * freqs[offset, :pairs]).flatten(-2).to(keys.dtype))
    return out


# ---------------------------------------------------------------- checks ----

def near_tie_rows(risk_, boundary, rel=1e-3):
    """Rows whose selection boundary is a near tie: the last kept and first
    dropped scores (in stable descending order) differ by at most `rel`
    relative.  boundary [H,T] = number kept from `risk_` (already restricted to
    the candidates, -inf elsewhere).  Returns bool [H,T]."""
    s = risk_.sort(dim=-1, descending=True).values
    idx = boundary.clamp(1, s.shape[-1] - 1).long()
    last = s.gather(-1, (idx - 1)[..., None])[..., 0]
    nxt = s.gather(-1, idx[..., None])[..., 0]
    scale = torch.maximum(last.abs(), nxt.abs())
    tie = (last - nxt).abs() <= rel * scale
    return tie & torch.isfinite(nxt)


def near_tie_order_rows(risk_, ids, start, rel=1e-3):
    """Rows whose risk-ordered LUT part ids[..., start:] holds two consecutive
    pages whose scores differ by at most `rel` relative: the order of those
    two is a rounding matter (it only changes the accumulation order of the
    attention that follows).  risk_ [H,T,P], ids [H,T,C].  Returns bool [H,T]."""
    r = risk_.gather(-1, ids[..., start:].long())
    a, b = r[..., :-1], r[..., 1:]
    scale = torch.maximum(a.abs(), b.abs())
    return ((a - b).abs() <= rel * scale).any(-1)


def rel_l2(a, b):
    a = a.double()
    b = b.double()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))
