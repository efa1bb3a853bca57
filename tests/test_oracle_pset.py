"""Pins the Full_Pset oracle (oracle/pset.py): swap gains against a direct
recomputation of the mixture after each swap, pools against the partition
rules, the readout and encodings against closed forms and torch.nn modules."""
import math

import pytest
import torch

from oracle import pset
from oracle import reference as ref
from streaming_sparse_amd import workload


def _mixture(logs, vals):
    w = logs.softmax(-1)
    return (w[..., None] * vals).sum(-2)


def _brute_scores(rp, beta, lm, cen, mask, remove, add):
    """Score of each swap from its definition: recompute the selected-page
    mixture after moving `remove` out and `add` in, then
    mean_m(2 E.(new-H) - |new-H|^2) with E = target - H."""
    b, m, p, _ = rp.shape
    le = lm + beta
    out = torch.empty(b, remove.shape[1], add.shape[1], dtype=torch.float64)
    for i in range(b):
        sel = mask[i]
        logs = torch.where(sel, le[i], lm[i])
        H = _mixture(logs, cen[i] + sel[None, :, None] * rp[i])
        target = _mixture(le[i], cen[i] + rp[i])
        E = target - H
        for x, r in enumerate(remove[i].tolist()):
            for y, a in enumerate(add[i].tolist()):
                s2 = sel.clone()
                s2[r] = False
                s2[a] = True
                logs2 = torch.where(s2, le[i], lm[i])
                new = _mixture(logs2, cen[i] + s2[None, :, None] * rp[i])
                d = new - H
                out[i, x, y] = (2 * (E * d).sum(-1) - d.square().sum(-1)).mean()
    return out


def _random_case(seed, b=2, m=3, p=14, big_beta=False):
    g = torch.Generator().manual_seed(seed)
    rp = torch.randn(b, m, p, 16, generator=g, dtype=torch.float64) * 0.3
    beta = torch.randn(b, m, p, generator=g, dtype=torch.float64) * 0.6      # both endpoint branches
    z = torch.randn(b, m, p, generator=g, dtype=torch.float64)
    lm = z - z.logsumexp(-1, keepdim=True)
    cen = torch.randn(b, m, p, 16, generator=g, dtype=torch.float64)
    mask = torch.zeros(b, p, dtype=torch.bool)
    mask[:, :6] = True
    remove = torch.tensor([[1, 3, 5], [0, 2, 4]])
    add = torch.tensor([[6, 9, 13, 7], [8, 10, 12, 11]])
    if big_beta:
        beta[:, :, 3] = 100.0          # removing page 3 drops its mass by e^100 -> "bad" path
        beta[:, :, 2] = -90.0
    return rp, beta, lm, cen, mask, remove, add


@pytest.mark.parametrize("seed,big", [(1, False), (2, False), (3, True)])
def test_grouped_scores_equal_direct_swap(seed, big):
    args = _random_case(seed, big_beta=big)
    got = pset.grouped_scores(*args)
    want = _brute_scores(*args)
    scale = want.abs().max()
    assert torch.isfinite(got).all()
    assert (got - want).abs().max() <= 1e-10 * scale + 1e-14, (got - want).abs().max()


def test_grouped_scores_no_effect_pair_is_zero():
    """A swap between two pages with identical log mass, beta = 0 and equal
    values changes nothing: gain exactly 0."""
    rp, beta, lm, cen, mask, remove, add = _random_case(4)
    beta[:, :, [1, 6]] = 0.0
    lm[:, :, 6] = lm[:, :, 1]
    cen[:, :, 6] = cen[:, :, 1]
    rp[:, :, 6] = rp[:, :, 1]
    got = pset.grouped_scores(rp, beta, lm, cen, mask, remove, add)
    assert abs(float(got[0, 0, 0])) < 1e-14


def _adversarial(p, rows, seed):
    g = torch.Generator().manual_seed(seed)
    out = torch.rand(rows, p, generator=g)
    out[0, ::3] = 0.0
    out[0, 1::3] = -0.0
    for i in range(1, rows):
        out[i] = torch.randint(0, [2, 7, 1000][i % 3], (p,), generator=g).float()
    return out


def _rule_pool(risk, sel, own, p):
    """Pool from its rules, one row, plain Python."""
    removes, adds, legal_r, legal_a = [], [], [], []
    for lo, hi in ((24, p - 72), (p - 72, p)):
        mov = [i for i in range(lo, hi) if sel[i] and i != own]
        uns = [i for i in range(lo, hi) if not sel[i]]
        mov.sort(key=lambda i: (float(risk[i]) + 0.0, i))
        uns.sort(key=lambda i: (-float(risk[i]) + 0.0, i))
        removes += [(mov[k], True) if k < len(mov) else (None, False) for k in range(8)]
        adds += [(uns[k], True) if k < len(uns) else (None, False) for k in range(16)]
    rm = [page if ok else slot for slot, (page, ok) in enumerate(removes)]
    valid_adds = {page for page, ok in adds if ok}
    spare = [i for i in range(p) if not sel[i] and i not in valid_adds]
    # past the spare pages a slot holds P (the reference's topk of a tensor filled with P)
    ad = [page if ok else (spare[slot] if slot < len(spare) else p) for slot, (page, ok) in enumerate(adds)]
    legal = [[removes[x][1] and adds[y][1] and ((x < 8) == (y < 16)) for y in range(32)] for x in range(16)]
    return rm, ad, legal


@pytest.mark.parametrize("p", [216, 432])
def test_pool_rules(p):
    h, t = 2, 4
    risk = _adversarial(p, h * t, 3).reshape(h, t, p)
    g = torch.Generator().manual_seed(9)
    mask = torch.rand(h, t, p, generator=g) < 0.12
    mask[..., :24] = True
    own = (torch.arange(t) + p - 72)[None].expand(h, -1).contiguous()
    mask.scatter_(-1, own[..., None], True)
    mask[1, 1, p - 72:] = True                  # current partition full: no adds there
    mask[1, 2, 24:p - 72] = False               # history partition empty: no removes there
    # nearly everything selected: 6 unselected current and 20 unselected
    # history pages leave 4 spare pages, and padded slot k takes spare k:
    # current slots 22..31 find none
    mask[0, 3] = True
    mask[0, 3, torch.arange(p - 72, p - 66)] = False
    mask[0, 3, torch.arange(24, 44)] = False
    r, a, legal = pset.pool(risk, mask, own)
    short = 0
    for hh in range(h):
        for tt in range(t):
            rm, ad, lg = _rule_pool(risk[hh, tt], mask[hh, tt].tolist(), int(own[hh, tt]), p)
            assert r[hh, tt].tolist() == rm
            assert a[hh, tt].tolist() == ad
            assert legal[hh, tt].tolist() == lg
            real = [x for x in rm + ad if x < p]
            assert len(set(real)) == len(real) and len(real) + ad.count(p) == 48
            short += ad.count(p)
    assert a[0, 3, 22:].tolist() == [p] * 10 and a[0, 3, :22].max() < p
    assert short == 10


def test_empty_add_slot_equals_a_spare_page():
    """An add slot past the spare pages holds page P, an empty candidate of
    zero mass (pool).  It scores every legal swap as a spare page in that
    slot does: a padded slot is an inactive add, and the reference's pool
    comment calls such pages equivalent background terms
    (VB/quota_pool.py:41-42).  Checked by moving a real spare page out of
    its slot (the page goes back to the background) and comparing all legal
    scores, and by the correction's decisions."""
    p, b, m = 216, 3, 4
    g = torch.Generator().manual_seed(21)
    risk = torch.rand(1, b, p, generator=g)
    mask = torch.rand(1, b, p, generator=g) < 0.5
    mask[..., :24] = True
    own = (torch.arange(b) + p - 72)[None].contiguous()
    mask.scatter_(-1, own[..., None], True)
    mask[0, :, p - 72:p - 62] = True             # 10 selected current pages at the partition start
    mask[0, :, p - 62:p - 52] = False
    mask[0, :, p - 52:] = True                   # 10 unselected current pages: 6 padded add slots
    r, a, legal = pset.pool(risk, mask, own)
    r, a, legal, mk = r[0], a[0], legal[0], mask[0]
    rp = torch.randn(b, m, p, 16, generator=g, dtype=torch.float64) * 0.3
    beta = torch.randn(b, m, p, generator=g, dtype=torch.float64) * 0.6
    z = torch.randn(b, m, p, generator=g, dtype=torch.float64)
    lm = z - z.logsumexp(-1, keepdim=True)
    cen = torch.randn(b, m, p, 16, generator=g, dtype=torch.float64)
    base = pset.grouped_scores(rp, beta, lm, cen, mk, r, a)
    padded = ~mk.gather(1, a) & ~legal.any(1)                 # spare pages in add slots (never legal)
    padded &= a < p
    assert int(padded.sum(-1).min()) >= 6
    emptied = torch.where(padded, p, a)
    got = pset.grouped_scores(rp, beta, lm, cen, mk, r, emptied)
    scale = base.masked_fill(~legal, 0).abs().amax()
    err = (got - base).abs().masked_fill(~legal, 0).amax()
    assert float(err) <= 1e-12 * float(scale), (float(err), float(scale))
    s0 = base.masked_fill(~legal, -1e30)
    s1 = got.masked_fill(~legal, -1e30)
    n0, _, e0, j0 = pset.apply_best(mk, r, a, s0)
    n1, _, e1, j1 = pset.apply_best(mk, r, emptied, s1)
    assert torch.equal(e0, e1) and torch.equal(j0, j1) and torch.equal(n0, n1)


def test_apply_best_leaves_rows_without_a_swap():
    """A row with no legal pair (or no gain) keeps its mask, even when its
    argmax names a padded slot holding a selected page or page P."""
    mask = torch.tensor([[True, True, False, True]])
    remove = torch.tensor([[1]])
    add = torch.tensor([[4, 3]])                 # page 4 = P (empty), page 3 selected
    scores = torch.full((1, 1, 2), -1e30, dtype=torch.float64)
    new, gain, executed, j = pset.apply_best(mask, remove, add, scores)
    assert not bool(executed[0]) and torch.equal(new, mask)


def _rule_pool72(risk, sel, own):
    """The first chunk's pool from its rules, one row of a 72-page window,
    plain Python: movable removes by (risk, page) up to 8, then the anchor
    pages other than own; adds by (-risk, page) over the unselected pages,
    then the selected pages by page; legal = movable x the first 16 adds."""
    mov = sorted((i for i in range(24, 72) if sel[i] and i != own), key=lambda i: (float(risk[i]) + 0.0, i))
    used = min(len(mov), 8)
    stand = [i for i in range(24) if i != own]
    rm = mov[:used] + stand[:16 - used]
    uns = sorted((i for i in range(72) if not sel[i]), key=lambda i: (-float(risk[i]) + 0.0, i))
    ad = (uns + [i for i in range(72) if sel[i]])[:32]
    legal = [[x < used and y < 16 for y in range(32)] for x in range(16)]
    return rm, ad, legal


def test_pool_rules_first_chunk():
    """72-page window (VB/quota_pool.py:21-33): rows with few and many
    movable pages, own inside and outside the anchor frame, fewer than 16
    and fewer than 32 unselected pages (the add slots then hold selected
    pages), signed-zero and integer-binned risks."""
    h, t, p = 2, 6, 72
    risk = _adversarial(p, h * t, 5).reshape(h, t, p)
    g = torch.Generator().manual_seed(11)
    mask = torch.rand(h, t, p, generator=g) < 0.4
    mask[..., :24] = True
    own = torch.tensor([[3, 30, 50, 71, 24, 0], [23, 40, 60, 25, 10, 70]])
    mask.scatter_(-1, own[..., None], True)
    mask[0, 1, 24:] = False
    mask[0, 1, 30] = True                       # only own beyond the anchors: no movable page
    mask[1, 2, 24:60] = True                    # 12 unselected pages: add slots 12..31 hold selected pages
    mask[1, 3, 24:] = True
    mask[1, 3, 60:64] = False                   # 4 unselected pages
    r, a, legal = pset.pool(risk, mask, own)
    for hh in range(h):
        for tt in range(t):
            rm, ad, lg = _rule_pool72(risk[hh, tt], mask[hh, tt].tolist(), int(own[hh, tt]))
            assert r[hh, tt].tolist() == rm
            assert a[hh, tt].tolist() == ad
            assert legal[hh, tt].tolist() == lg
            assert len(set(rm)) == 16 and len(set(ad)) == 32


def test_read_closed_forms():
    g = torch.Generator().manual_seed(4)
    h, t, m, p = 2, 2, 3, 5
    probes = torch.randn(h, t, m, 128, generator=g)
    co = torch.randn(h, p, 5, 17, generator=g).bfloat16()
    wq = torch.randn(8, 128, generator=g) * 0.02
    # A = 0 -> F = 0 -> value = co row 0
    rp, beta = pset.read(probes, co, torch.zeros(h, p, 8, 4), wq)
    torch.testing.assert_close(rp, co.float()[:, None, None, :, 0, :16].expand_as(rp))
    torch.testing.assert_close(beta, co.float()[:, None, None, :, 0, 16].expand_as(beta))
    # u_0 * A[0,j] = atanh(0.5) for j = 2 only -> value = co0 + 0.5 co3
    u0 = probes @ wq.t()
    a = torch.zeros(h, p, 8, 4)
    a[..., 0, 2] = 1.0
    probes2 = probes.clone()
    scale = math.atanh(0.5) / u0[..., 0]
    rp2, beta2 = pset.read(probes2 * scale[..., None], co, a, wq)
    want = co.float()[:, None, None, :, 0] + 0.5 * co.float()[:, None, None, :, 3]
    torch.testing.assert_close(rp2, want[..., :16].expand_as(rp2), atol=2e-5, rtol=1e-5)
    torch.testing.assert_close(beta2, want[..., 16].expand_as(beta2), atol=2e-5, rtol=1e-5)


def test_encode_matches_torch_modules():
    """co / A equal nn.Sequential(Linear, GELU, Linear) of the same weights on
    the normalised features; features have RMS rms/(rms+1e-4) per part."""
    h, p = 2, 6
    g = torch.Generator().manual_seed(8)
    k = torch.randn(h, p, 64, 128, generator=g).bfloat16()
    v = torch.randn(h, p, 64, 128, generator=g).bfloat16()
    basis = workload.pca_basis(v.float())
    s = workload.kmeans_summaries(k, v, basis, torch.Generator().manual_seed(1))
    w = workload.reader_weights()
    enc = pset.encode(s.keys, s.mean, s.detail, s.stats, basis, w)
    f = pset.page_features(s.keys, s.mean, s.detail, s.stats)
    assert f.shape == (h, p, 712)
    for lo, hi, x in ((0, 512, s.keys.float().flatten(2)), (512, 640, s.mean.float()),
                      (640, 664, s.detail.float().flatten(2)), (664, 712, s.stats.float().flatten(2))):
        rms = x.square().mean(-1).sqrt()
        torch.testing.assert_close(f[..., lo:hi].square().mean(-1).sqrt(), rms / (rms + 1e-4))
    for name, out, shape in (('reader', 85, (5, 17)), ('phi', 32, (8, 4))):
        net = torch.nn.Sequential(torch.nn.Linear(712, 256), torch.nn.GELU(), torch.nn.Linear(256, out))
        with torch.no_grad():
            net[0].weight.copy_(w[name + '_w1'])
            net[0].bias.copy_(w[name + '_b1'])
            net[2].weight.copy_(w[name + '_w2'])
            net[2].bias.copy_(w[name + '_b2'])
            want = net(f).reshape(h, p, *shape).bfloat16()
        got = enc['co'] if name == 'reader' else enc['A']
        assert torch.equal(got, want)
    bas = basis.bfloat16().double()
    want_detail = torch.einsum('hpak,hdk,de->hpae', s.detail.double(), bas, w['B'])
    torch.testing.assert_close(enc['detail'], want_detail, atol=1e-12, rtol=1e-12)
    torch.testing.assert_close(enc['mean'], s.mean.double() @ w['B'], atol=1e-12, rtol=1e-12)


def test_log_mass_and_center():
    g = torch.Generator().manual_seed(2)
    z = torch.zeros(1, 2, 3, 10, 4)
    lm = pset.log_mass(z)
    torch.testing.assert_close(lm, torch.full_like(lm, -math.log(10)))
    z = torch.randn(1, 2, 3, 10, 4, generator=g) * 3
    lm = pset.log_mass(z)
    torch.testing.assert_close(lm.logsumexp(-1), torch.zeros(1, 2, 3, dtype=torch.float64), atol=1e-12, rtol=0)
    mean_b = torch.randn(1, 10, 16, generator=g, dtype=torch.float64)
    detail_b = torch.randn(1, 10, 3, 16, generator=g, dtype=torch.float64)
    c = pset.center(z, lm, mean_b, detail_b)
    torch.testing.assert_close((lm.exp()[..., None] * c).sum(-2), torch.zeros(1, 2, 3, 16, dtype=torch.float64),
                               atol=1e-12, rtol=0)
    # equal rep logits -> zero Haar contrasts -> approx = meanB
    c0 = pset.center(torch.zeros(1, 1, 1, 10, 4), pset.log_mass(torch.zeros(1, 1, 1, 10, 4)), mean_b, detail_b)
    torch.testing.assert_close(c0[0, 0, 0], mean_b[0] - mean_b[0].mean(0), atol=1e-12, rtol=0)


def test_apply_best():
    mask = torch.tensor([[True, True, False, False]] * 3)
    remove = torch.tensor([[0, 1]] * 3)
    add = torch.tensor([[2, 3]] * 3)
    scores = torch.tensor([[[-1.0, -2.0], [-0.5, -3.0]],
                           [[-1.0, 0.2], [0.7, -3.0]],
                           [[-1.0, 0.2], [0.7, math.nan]]], dtype=torch.float64)
    new, gain, executed, j = pset.apply_best(mask, remove, add, scores)
    assert new[0].tolist() == [True, True, False, False] and not executed[0]
    assert new[1].tolist() == [True, False, True, False] and executed[1] and int(j[1]) == 2
    assert new[2].tolist() == [True, True, False, False] and not executed[2]


def test_correct_pipeline_invariants():
    """Config-3-shaped rows at P=216, 2 of 3 heads scoped: quota counts are
    preserved per partition, anchors and own stay, an executed row differs by
    one same-partition swap whose gain is the direct recomputation."""
    x = workload.make_call(cfg=3, frames=9, heads=3)
    w = workload.reader_weights()
    pr = ref.probes(x.q)
    z = ref.route_logits(pr, x.summary.keys)
    r = ref.risk(pr, z, x.summary.stats, x.theta)
    a = torch.tensor([8, 18, 4])
    n = 20
    mask = ref.quota_mask(r, x.own, a, n)
    enc = pset.encode(x.summary.keys, x.summary.mean, x.summary.detail, x.summary.stats, x.basis, w)
    new, rows, stats = pset.correct(pr.bfloat16().float(), z, r, mask, x.own, enc, w['wq'], [0, 2])
    p = x.pages
    assert torch.equal(new[1], mask[1])
    assert int(stats[1]) == 2 * 72 and int(stats[2]) == 0
    for hi, hh in enumerate([0, 2]):
        for t in range(72):
            old, cur = mask[hh, t], new[hh, t]
            assert cur[:24].all() and cur[x.own[hh, t]]
            assert int(cur[p - 72:].sum()) == int(a[hh]) and int(cur[24:p - 72].sum()) == n - int(a[hh])
            changed = (old != cur).nonzero().flatten().tolist()
            if rows['executed'][hi, t]:
                assert len(changed) == 2
            else:
                assert changed == []
    # the executed gain is the direct recomputation for one executed row
    hi, t = [(i, j) for i in range(2) for j in range(72) if rows['executed'][i, j]][0]
    j = int(rows['argmax'][hi, t])
    rr, aa = rows['remove'][hi, t, j // 32], rows['add'][hi, t, j % 32]
    b = lambda v: v[hi, t][None]
    want = _brute_scores(b(rows['rp']).double(), b(rows['beta']).double(), b(rows['lm']), b(rows['center']),
                         mask[[0, 2][hi], t][None], rr.reshape(1, 1), aa.reshape(1, 1))
    torch.testing.assert_close(rows['gain'][hi, t], want[0, 0, 0], atol=1e-12, rtol=1e-9)
    assert int(stats[0]) == int(rows['executed'].sum()) > 0
