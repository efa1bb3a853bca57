"""Full_Pset on the HIP path vs. the CPU oracle (oracle/pset.py) on identical
seeded inputs: config-3 shapes (432-page window, intersection quotas,
heads {3,4,9}).

Bar: encodings bit-exact except isolated 1-ulp bf16 roundings of the MLP
outputs; swap scores within 1e-4 of the row's score scale; executed swaps and
the final masks identical except rows whose decision is a near tie (best and
second-best legal gain, or the best gain and 0, within 1e-3 relative)."""
import functools
import math

import pytest
import torch

from oracle import pset as opset
from oracle import reference as ref
from streaming_sparse_amd import pset, workload
from streaming_sparse_amd.attention import Workspace
from streaming_sparse_amd.route import route

pytestmark = pytest.mark.gpu
HEADS = [3, 4, 9]


@functools.lru_cache(maxsize=None)
def inputs(frames=18):
    x = workload.make_call(cfg=3, frames=frames)
    w = workload.reader_weights()
    tab = workload.quota_table(3)
    a = tab[0, 3, :, 0]
    n = int(tab[0, 3, 0].sum())
    return x, w, a, n


def gpu_encoding(x, w, device):
    g = x.to(device)
    reader = pset.Reader(w, device)
    enc = pset.encode(g.summary, g.basis, reader)
    torch.cuda.synchronize()
    return g, reader, enc


def test_encode_matches_oracle(device):
    x, w, _, _ = inputs(9)
    _, _, enc = gpu_encoding(x, w, device)
    want = opset.encode(x.summary.keys, x.summary.mean, x.summary.detail, x.summary.stats, x.basis, w)
    for name, got in (('co', enc.co.cpu()), ('A', enc.A.cpu())):
        ref_v = want[name]
        diff = got != ref_v
        frac = float(diff.float().mean())
        # an fp32 accumulation-order difference moves a value across a bf16
        # rounding boundary: one bf16 ulp (at most 2^-7 relative), or a few
        # ulps of a value that cancelled to near zero
        err = (got.float() - ref_v.float()).abs()
        bound = ref_v.float().abs() * 2.0 ** -7 + 1e-6
        print(f"{name}: {int(diff.sum())} of {diff.numel()} bf16 values differ, max abs {float(err.max()):.2e}",
              flush=True)
        assert bool((err <= bound).all()) and frac < 1e-3
    torch.testing.assert_close(enc.mean.cpu(), want['mean'], atol=1e-12, rtol=1e-12)
    torch.testing.assert_close(enc.detail.cpu(), want['detail'], atol=1e-12, rtol=1e-12)
    assert (enc.coef[..., 85:96] == 0).all()


def _near_tie(scores, legal, rel=1e-3):
    """Rows whose decision is fragile: best two legal scores, or the best
    score and 0, within `rel` of the row's score scale."""
    s = scores.masked_fill(~legal, -math.inf).flatten(-2)
    top = s.topk(2, dim=-1).values
    scale = s.masked_fill(~legal.flatten(-2), 0).abs().amax(-1).clamp_min(1e-300)
    return ((top[..., 0] - top[..., 1]).abs() <= rel * scale) | (top[..., 0].abs() <= rel * scale)


@pytest.mark.parametrize("frames", [18, 12])
def test_pset_matches_oracle(device, frames):
    x, w, a, n = inputs(frames)
    g, reader, enc = gpu_encoding(x, w, device)
    ws = Workspace()
    lse = torch.empty(12, 72, 16, device=device)
    ids, mask, risk, _ = route(g.q, g.summary, g.theta, tier='intersection', own=g.own, current_slots=a, n=n,
                               workspace=ws, lse_out=lse)
    mask0 = mask.clone()
    ids0 = ids.clone()
    stats, rows = pset.correct(g.q, g.summary, enc, reader, risk, lse, mask, ids, g.own, HEADS, want_scores=True)
    torch.cuda.synchronize()
    # oracle on the same selection, risk and encodings
    pr = ref.probes(x.q)
    z = ref.route_logits(pr, x.summary.keys)
    want_lse = ref.route_logits(pr, x.summary.keys, torch.float64).flatten(-2).logsumexp(-1)
    lse_err = float((lse.cpu().double() - want_lse).abs().max())
    print(f"probe lse max abs err {lse_err:.2e}", flush=True)
    assert lse_err < 1e-5
    enc_o = dict(co=enc.co.cpu(), A=enc.A.cpu(), mean=enc.mean.cpu(), detail=enc.detail.cpu())
    m0 = mask0.cpu()
    want_mask, orow, ostats = opset.correct(pr.bfloat16().float(), z, risk.cpu(), m0, x.own, enc_o, w['wq'], HEADS)
    legal = orow['legal'].reshape(len(HEADS), 72, 16, 32)
    got_s = rows['scores'].cpu()
    want_s = orow['scores']
    scale = want_s.masked_fill(~legal, 0).abs().flatten(-2).amax(-1).clamp_min(1e-300)
    err = ((got_s - want_s).abs().masked_fill(~legal, 0).flatten(-2).amax(-1) / scale)
    print(f"scores: max err / row scale {float(err.max()):.2e}; gpu executed {int(stats[0])}, "
          f"oracle executed {int(ostats[0])} of {int(ostats[1])}", flush=True)
    assert float(err.max()) < 1e-4
    assert (got_s.masked_fill(legal, 0) == -1e30).masked_fill(legal, True).all()
    pool = rows['pool'].cpu()
    assert torch.equal(pool[..., :16].long(), orow['remove'])
    assert torch.equal(pool[..., 16:48].long(), orow['add'])
    ties = _near_tie(want_s, legal)
    ex_g = rows['executed'].cpu().bool()
    same = (ex_g == orow['executed']) & (~ex_g | (rows['argmax'].cpu().long() == orow['argmax']))
    print(f"decisions: {int(same.sum())}/{same.numel()} identical, {int(ties.sum())} near-tie rows", flush=True)
    assert bool((same | ties).all())
    got_mask = mask.cpu()
    hs = torch.tensor(HEADS)
    rows_equal = (got_mask[hs] == want_mask[hs]).all(-1)
    assert bool((rows_equal | ties).all())
    others = [i for i in range(12) if i not in HEADS]
    assert torch.equal(got_mask[others], m0[others]) and torch.equal(ids.cpu()[others], ids0.cpu()[others])
    # LUT of every corrected row: own first, exactly the new mask, descending risk
    got_ids = ids.cpu()
    assert torch.equal(ref.mask_from_ids(got_ids, x.pages), got_mask)
    assert (got_ids[..., 0] == x.own).all()
    rk = risk.cpu().gather(-1, got_ids[..., 1:].long())
    assert (rk[..., :-1] >= rk[..., 1:]).all()
    # quotas survive the swaps
    assert (got_mask[..., x.pages - 72:].sum(-1) == a[:, None]).all()
    assert (got_mask[..., :24]).all()


def test_route_full_pset_end_to_end(device):
    """route(..., full_pset=heads) against the oracle chain risk (fp64) ->
    quota mask -> Full_Pset, on rows that are not near ties at either step."""
    x, w, a, n = inputs()
    g, reader, enc = gpu_encoding(x, w, device)
    ids, mask, risk, stats = route(g.q, g.summary, g.theta, tier='intersection', own=g.own, current_slots=a, n=n,
                                   full_pset=HEADS, encoding=enc, reader=reader)
    torch.cuda.synchronize()
    pr = ref.probes(x.q)
    z = ref.route_logits(pr, x.summary.keys)
    r64 = ref.risk(pr, ref.route_logits(pr, x.summary.keys, torch.float64), x.summary.stats, x.theta,
                   dtype=torch.float64)
    m0 = ref.quota_mask(r64, x.own, a, n)
    enc_o = dict(co=enc.co.cpu(), A=enc.A.cpu(), mean=enc.mean.cpu(), detail=enc.detail.cpu())
    want, orow, _ = opset.correct(pr.bfloat16().float(), z, r64.float(), m0, x.own, enc_o, w['wq'], HEADS)
    P = x.pages
    hist = r64.clone()
    hist[..., :24] = -math.inf
    hist[..., P - 72:] = -math.inf
    cur = r64.clone()
    cur[..., :P - 72] = -math.inf
    cur.scatter_(-1, x.own[..., None], math.inf)
    route_ties = ref.near_tie_rows(hist, (n - a)[:, None].expand_as(x.own)) | \
        ref.near_tie_rows(cur, a[:, None].expand_as(x.own))
    hs = torch.tensor(HEADS)
    ties = route_ties.clone()
    ties[hs] |= _near_tie(orow['scores'], orow['legal'].reshape(len(HEADS), 72, 16, 32))
    same = (mask.cpu() == want).all(-1)
    print(f"end to end: {int(same.sum())}/{same.numel()} masks identical, {int(ties.sum())} near-tie rows, "
          f"executed {int(stats[0])}/{int(stats[1])}", flush=True)
    assert bool((same | ties).all())
    assert int(stats[1]) == len(HEADS) * 72 and int(stats[2]) == 0


@pytest.mark.parametrize("n", [4, 20, 40])
def test_pset_first_chunk_matches_oracle(device, n):
    """Full_Pset on a 72-page window, the first chunk's (VB/quota_pool.py:
    21-33): the anchor frame is the chunk's first frame, own page t of block
    t.  n = 4 is the reference's first-chunk quota (VB/queue_policy.py:26);
    n = 20 leaves 28 unselected pages, so add slots 28..31 hold selected
    (anchor) pages, also listed as remove stand-ins; n = 40 leaves 8, so
    legal adds hold selected pages too.  Pools equal, scores within 1e-4 of
    the row scale, decisions and masks equal off near ties."""
    x = workload.make_call(cfg=3, frames=3)
    w = workload.reader_weights()
    assert x.pages == 72
    g, reader, enc = gpu_encoding(x, w, device)
    ws = Workspace()
    lse = torch.empty(12, 72, 16, device=device)
    ids, mask, risk, _ = route(g.q, g.summary, g.theta, tier='intersection', own=g.own, n=n, workspace=ws,
                               lse_out=lse)
    mask0 = mask.clone()
    stats, rows = pset.correct(g.q, g.summary, enc, reader, risk, lse, mask, ids, g.own, HEADS, want_scores=True)
    torch.cuda.synchronize()
    pr = ref.probes(x.q)
    z = ref.route_logits(pr, x.summary.keys)
    enc_o = dict(co=enc.co.cpu(), A=enc.A.cpu(), mean=enc.mean.cpu(), detail=enc.detail.cpu())
    m0 = mask0.cpu()
    assert (m0.sum(-1) == 24 + n).all()
    want_mask, orow, ostats = opset.correct(pr.bfloat16().float(), z, risk.cpu(), m0, x.own, enc_o, w['wq'], HEADS)
    pool = rows['pool'].cpu()
    assert torch.equal(pool[..., :16].long(), orow['remove'])
    assert torch.equal(pool[..., 16:48].long(), orow['add'])
    legal = orow['legal'].reshape(len(HEADS), 72, 16, 32)
    got_s = rows['scores'].cpu()
    want_s = orow['scores']
    scale = want_s.masked_fill(~legal, 0).abs().flatten(-2).amax(-1).clamp_min(1e-300)
    err = ((got_s - want_s).abs().masked_fill(~legal, 0).flatten(-2).amax(-1) / scale)
    print(f"n={n}: scores max err / row scale {float(err.max()):.2e}; gpu executed {int(stats[0])}, "
          f"oracle executed {int(ostats[0])} of {int(ostats[1])}", flush=True)
    assert float(err.max()) < 1e-4
    assert (got_s.masked_fill(legal, 0) == -1e30).masked_fill(legal, True).all()
    ties = _near_tie(want_s, legal)
    ex_g = rows['executed'].cpu().bool()
    same = (ex_g == orow['executed']) & (~ex_g | (rows['argmax'].cpu().long() == orow['argmax']))
    print(f"decisions: {int(same.sum())}/{same.numel()} identical, {int(ties.sum())} near-tie rows", flush=True)
    assert bool((same | ties).all())
    got_mask = mask.cpu()
    hs = torch.tensor(HEADS)
    assert bool(((got_mask[hs] == want_mask[hs]).all(-1) | ties).all())
    # the LUT of every row: own first, then the selection by descending risk, -1 past its end
    got_ids = ids.cpu()
    assert torch.equal(ref.mask_from_ids(got_ids, 72), got_mask)
    assert (got_ids[..., 0] == x.own).all() and got_mask[..., :24].all()
    want_ids = ref.lut(risk.cpu(), got_mask, x.own, 24 + n)
    assert torch.equal(got_ids.sort(-1).values, want_ids.sort(-1).values)


def test_pset_short_spares_matches_oracle(device):
    """A table too full for the stratified pool's spare pages: 216-page
    window, A = 66 of 72 current and B = 100 of 120 history pages (190 of
    216 selected).  Each row has 6 unselected current and 20 unselected
    history pages, so padded current add slot k (22..31) finds no spare page
    k and is an empty candidate: -1 in the pool, P in the oracle's (the
    reference's spare fill value), zero mass in the scores.  Pools equal
    (P -> -1), scores within 1e-4 of the row scale, decisions and masks
    equal off near ties."""
    x = workload.make_call(cfg=3, frames=9)
    w = workload.reader_weights()
    P = x.pages
    a = torch.full((12,), 66, dtype=torch.int32)
    n = 166
    g, reader, enc = gpu_encoding(x, w, device)
    ws = Workspace()
    lse = torch.empty(12, 72, 16, device=device)
    ids, mask, risk, _ = route(g.q, g.summary, g.theta, tier='intersection', own=g.own, current_slots=a, n=n,
                               workspace=ws, lse_out=lse)
    mask0 = mask.clone()
    stats, rows = pset.correct(g.q, g.summary, enc, reader, risk, lse, mask, ids, g.own, HEADS, want_scores=True)
    torch.cuda.synchronize()
    pr = ref.probes(x.q)
    z = ref.route_logits(pr, x.summary.keys)
    enc_o = dict(co=enc.co.cpu(), A=enc.A.cpu(), mean=enc.mean.cpu(), detail=enc.detail.cpu())
    m0 = mask0.cpu()
    assert (m0.sum(-1) == 24 + n).all()
    want_mask, orow, ostats = opset.correct(pr.bfloat16().float(), z, risk.cpu(), m0, x.own, enc_o, w['wq'], HEADS)
    pool = rows['pool'].cpu()
    want_add = orow['add'].masked_fill(orow['add'] == P, -1)
    assert int((want_add == -1).sum()) >= 10 * len(HEADS) * 72
    assert torch.equal(pool[..., :16].long(), orow['remove'])
    assert torch.equal(pool[..., 16:48].long(), want_add)
    legal = orow['legal'].reshape(len(HEADS), 72, 16, 32)
    got_s = rows['scores'].cpu()
    want_s = orow['scores']
    assert torch.isfinite(want_s.masked_fill(~legal, 0)).all()
    scale = want_s.masked_fill(~legal, 0).abs().flatten(-2).amax(-1).clamp_min(1e-300)
    err = ((got_s - want_s).abs().masked_fill(~legal, 0).flatten(-2).amax(-1) / scale)
    print(f"short spares: scores max err / row scale {float(err.max()):.2e}; gpu executed {int(stats[0])}, "
          f"oracle executed {int(ostats[0])} of {int(ostats[1])}", flush=True)
    assert float(err.max()) < 1e-4
    assert int(stats[2]) == 0
    ties = _near_tie(want_s, legal)
    ex_g = rows['executed'].cpu().bool()
    same = (ex_g == orow['executed']) & (~ex_g | (rows['argmax'].cpu().long() == orow['argmax']))
    assert bool((same | ties).all())
    hs = torch.tensor(HEADS)
    got_mask = mask.cpu()
    assert bool(((got_mask[hs] == want_mask[hs]).all(-1) | ties).all())
    assert (got_mask[..., P - 72:].sum(-1) == 66).all() and got_mask[..., :24].all()
