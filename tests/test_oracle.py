"""Pins the CPU oracle (oracle/reference.py) against closed forms, brute force
and the reference's own CPU contracts (local_experiments/review_v1/test_ops.py),
before it is trusted to judge the HIP path."""
import math

import pytest
import torch

from oracle import reference as ref
from streaming_sparse_amd.ops import Summary
from streaming_sparse_amd import workload


def _tiny(h=2, p=6, n=64, seed=192):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, n, h, 128, generator=g).bfloat16()
    k = torch.randn(1, 64 * p, h, 128, generator=g).bfloat16()
    v = (torch.randn(1, 64 * p, h, 128, generator=g) + 0.5).bfloat16()
    kp = k[0].transpose(0, 1).reshape(h, p, 64, 128)
    vp = v[0].transpose(0, 1).reshape(h, p, 64, 128)
    basis = workload.pca_basis(vp.float())
    s = workload.kmeans_summaries(kp, vp, basis, torch.Generator().manual_seed(seed + 1))
    return q, k, v, s, basis


def test_all_selected_equals_dense():
    """All pages exact == softmax attention (RV/test_ops.py:19-23)."""
    q, k, v, s, basis = _tiny()
    h, p = 2, 6
    ids = torch.arange(p).expand(h, 1, p).int()
    out = ref.selected_attention(q, k, v, s, basis, ids)
    dense = torch.nn.functional.scaled_dot_product_attention(
        q[0].transpose(0, 1).float(), k[0].transpose(0, 1).float(), v[0].transpose(0, 1).float())
    torch.testing.assert_close(out[0].transpose(0, 1), dense, atol=2e-6, rtol=2e-6)
    torch.testing.assert_close(ref.dense_attention(q, k, v), out, atol=2e-6, rtol=2e-6)


def test_zero_query_closed_form():
    """q = 0: exact part = mean of selected tokens' V, tail = mean of the
    unselected page means (Haar contrasts of equal weights vanish), merged by
    token counts 64*C : 64*(P-C) (RV/test_ops.py:14-18 for the all-unselected
    case)."""
    q, k, v, s, basis = _tiny()
    q = torch.zeros_like(q)
    h, p = 2, 6
    ids = torch.tensor([[[5, 1]], [[4, 0]]], dtype=torch.int32)
    out = ref.selected_attention(q, k, v, s, basis, ids)
    vp = v[0].transpose(0, 1).reshape(h, p, 64, 128).float()
    for hh in range(h):
        sel = ids[hh, 0].long()
        uns = [i for i in range(p) if i not in sel.tolist()]
        exact = vp[hh, sel].reshape(-1, 128).mean(0)
        tail = s.mean[hh, uns].float().mean(0)
        expect = (len(sel) * exact + len(uns) * tail) / p
        torch.testing.assert_close(out[0, :, hh], expect.expand(64, -1), atol=2e-6, rtol=2e-6)


def _union_softmax_fp64(q, k, v, s, basis, ids):
    """Independent float64 statement of the call: one softmax over the exact
    tokens (logit q.k/sqrt(D), value v) and the reps of unselected pages (logit
    q.r/sqrt(D) + log 16, value mean_p + sum_a HAAR[a,r] detail_pa . basis^T)."""
    _, n, h, d = q.shape
    p = k.shape[1] // 64
    out = torch.zeros(h, n, d, dtype=torch.float64)
    ha = torch.tensor(ref.HAAR, dtype=torch.float64)
    bas = basis.bfloat16().double()
    for hh in range(h):
        for t in range(n // 64):
            sel = set(ids[hh, t].tolist())
            qq = q[0, t * 64:(t + 1) * 64, hh].double()
            logits, vals = [], []
            for page in range(p):
                if page in sel:
                    kk = k[0, page * 64:(page + 1) * 64, hh].double()
                    logits.append(qq @ kk.T / math.sqrt(d))
                    vals.append(v[0, page * 64:(page + 1) * 64, hh].double())
                else:
                    rk = s.keys[hh, page].double()
                    logits.append(qq @ rk.T / math.sqrt(d) + math.log(16))
                    code = ha.T @ s.detail[hh, page].double()          # [4 reps, 8]
                    vals.append(s.mean[hh, page].double()[None] + code @ bas[hh].T)
            z = torch.cat(logits, 1)
            w = torch.softmax(z, 1)
            out[hh, t * 64:(t + 1) * 64] = w @ torch.cat(vals, 0)
    return out.transpose(0, 1)[None]


def test_union_softmax_brute_force():
    q, k, v, s, basis = _tiny(h=2, p=7, n=128, seed=5)
    ids = torch.tensor([[[6, 0, 3], [5, 1, 2]], [[6, 4, 2], [5, 0, 1]]], dtype=torch.int32)
    got = ref.selected_attention(q, k, v, s, basis, ids, dtype=torch.float64)
    want = _union_softmax_fp64(q, k, v, s, basis, ids)
    torch.testing.assert_close(got, want, atol=1e-10, rtol=1e-10)
    got32 = ref.selected_attention(q, k, v, s, basis, ids)
    assert ref.rel_l2(got32, want) < 1e-5


def test_risk_zero_query():
    """Zero query: features 1..3 vanish and feature 0 = stats[p,0,11]/P
    (RV/test_ops.py:32-38 with all pages valid)."""
    _, _, _, s, _ = _tiny(p=5)
    q = torch.zeros(2, 4, 128)
    f, logz = ref.route_features(q, s.keys, s.stats)
    torch.testing.assert_close(f[..., 1:], torch.zeros_like(f[..., 1:]))
    expect = s.stats[:, :, 0, 11].float() / 5
    torch.testing.assert_close(f[..., 0], expect[:, None].expand(2, 4, 5))
    torch.testing.assert_close(logz, torch.full_like(logz, math.log(20)))
    pr = torch.zeros(2, 1, 16, 128)
    theta = torch.tensor([[0.7, 1, 1, 0.5], [1.3, 1, 1, 0.5]])
    z = ref.route_logits(pr, s.keys)
    r = ref.risk(pr, z, s.stats, theta)
    torch.testing.assert_close(r[:, 0], theta[:, :1] * expect)


def test_risk_scalar_brute_force():
    """Scalar restatement of the four features, loop by loop, in float64."""
    _, _, _, s, _ = _tiny(h=1, p=3, seed=11)
    g = torch.Generator().manual_seed(3)
    pr = torch.randn(1, 1, 16, 128, generator=g).bfloat16().float()
    theta = torch.tensor([[0.9, 1.1, 0.8, 0.5]])
    z = ref.route_logits(pr, s.keys, dtype=torch.float64)
    got = ref.risk(pr, z, s.stats, theta, dtype=torch.float64)
    st = s.stats.double()[0]
    keys = s.keys.double()[0]
    P = 3
    bmax = max(float(st[p, 1, 11]) for p in range(P))
    want = [0.0] * P
    for m in range(16):
        q = pr[0, 0, m].double()
        zz = [[float(q @ keys[p, r]) / math.sqrt(128) for r in range(4)] for p in range(P)]
        mx = max(max(row) for row in zz)
        den = sum(math.exp(x - mx) for row in zz for x in row)
        q2 = [float(q[16 * g_:16 * g_ + 16].square().sum()) / 128 for g_ in range(8)]
        qn = float(q.norm()) / math.sqrt(128)
        for p in range(P):
            prob = [math.exp(x - mx) / den for x in zz[p]]
            alpha = sum(prob)
            c = float(st[p, 1, 11]) + bmax
            x0 = alpha * float(st[p, 0, 11])
            x1 = x2 = x3 = 0.0
            for r in range(4):
                u = max(0.0, sum(q2[g_] * float(st[p, r, g_]) for g_ in range(8)))
                beta = qn * float(st[p, r, 8])
                x0 += abs(prob[r] - alpha / 4) * float(st[p, r, 9])
                x1 += prob[r] * math.sqrt(u) * float(st[p, r, 10])
                x2 += c * prob[r] * beta
                x3 += c * prob[r] * (u + beta * beta)
            th = theta[0].double().tolist()
            want[p] += (th[0] * x0 + th[1] * x1 + th[2] * x2 + th[3] * x3) / 16
    torch.testing.assert_close(got[0, 0], torch.tensor(want, dtype=torch.float64), atol=1e-12, rtol=1e-10)
    # the deployed form equals the RouteOps feature form averaged over probes
    f, _ = ref.route_features(pr[:, 0], s.keys, s.stats, dtype=torch.float64)
    alt = (f * theta.double()[:, None, None]).sum(-1).mean(1)
    torch.testing.assert_close(got[:, 0], alt, atol=1e-12, rtol=1e-10)


def _adversarial_rows(p, rows, seed):
    """Risk rows with heavy ties: signed zeros at strides 2/3/9/47 and integer
    bins, after local_experiments/video_runtime_v1/check_fixed_page_select.py:32-37."""
    g = torch.Generator().manual_seed(seed)
    out = torch.rand(rows, p, generator=g)
    for i, stride in enumerate((2, 3, 9, 47)):
        r = out[i % rows]
        r[::stride] = 0.0
        r[1::stride] = -0.0
    for i in range(4, rows):
        bins = [1, 2, 7, 1000, 1_000_000][i % 5]
        out[i] = torch.randint(0, bins, (p,), generator=g).float()
    return out


def _brute_top(scores, cand, k):
    """Top-k candidates by (score desc, index asc) with -0.0 == +0.0."""
    order = sorted(cand, key=lambda i: (-float(scores[i]) + 0.0, i))
    return order[:k]


@pytest.mark.parametrize("p", [216, 432])
def test_select_base_semantics(p):
    h, t = 2, 8
    risk = _adversarial_rows(p, h * t, 7).reshape(h, t, p)
    own = (torch.arange(t) + p - 72)[None].expand(h, -1).contiguous()
    count = p * 15 // 100
    ids = ref.select_base(risk, own, count)
    for hh in range(h):
        for tt in range(t):
            row = ids[hh, tt].tolist()
            assert row[0] == own[hh, tt] and row[1:25] == list(range(24))
            cand = [i for i in range(24, p) if i != own[hh, tt]]
            assert row[25:] == _brute_top(risk[hh, tt], cand, count - 25)


@pytest.mark.parametrize("p", [216, 432])
def test_quota_mask_semantics(p):
    h, t = 3, 6
    risk = _adversarial_rows(p, h * t, 9).reshape(h, t, p)
    own = (torch.arange(t) + p - 72)[None].expand(h, -1).contiguous()
    current = torch.tensor([1, 17, 36])
    total = 40
    mask = ref.quota_mask(risk, own, current, total)
    count = 24 + total
    ids = ref.lut(risk, mask, own, count)
    for hh in range(h):
        a = int(current[hh])
        for tt in range(t):
            m = mask[hh, tt]
            assert m[:24].all() and int(m[p - 72:].sum()) == a and bool(m[own[hh, tt]])
            assert int(m[24:p - 72].sum()) == total - a
            hist = _brute_top(risk[hh, tt], range(24, p - 72), total - a)
            assert sorted(hist) == [i for i in range(24, p - 72) if m[i]]
            r = risk[hh, tt].clone()
            r[own[hh, tt]] = torch.inf
            cur = _brute_top(r, range(p - 72, p), a)
            assert sorted(cur) == [i for i in range(p - 72, p) if m[i]]
            # LUT: own first, exactly the mask, then descending risk (queue audit
            # invariants of VB/queue_policy.py:42-44)
            row = ids[hh, tt].tolist()
            assert row[0] == own[hh, tt] and len(set(row)) == count
            assert sorted(row) == [i for i in range(p) if m[i]]
            rest = [i for i in range(p) if m[i] and i != own[hh, tt]]
            assert row[1:] == _brute_top(risk[hh, tt], rest, count - 1)


@pytest.mark.parametrize("p", [72, 96, 216])
def test_quota_mask_clamped_and_first_chunk(p):
    """Quotas outside their partitions and the first-chunk window, against a
    plain-Python restatement of _keep (VB/quota_mask.py:7-15: slots <= 0
    keeps nothing, slots >= the partition keeps all of it; the history quota
    is TOTAL - current with the unclamped current, :25), of the 72-page
    branch (VB/graph.py:143-148) and of the final topk LUT (VB/graph.py:210)
    with -1 where topk would run into unselected pages."""
    h, t = 5, 6
    risk = _adversarial_rows(p, h * t, 11).reshape(h, t, p)
    if p == 72:
        own = torch.tensor([3, 23, 24, 40, 60, 71])[None].expand(h, -1).contiguous()
        total = 30
    else:
        own = (torch.arange(t) * 13 % 72 + p - 72)[None].expand(h, -1).contiguous()
        total = {96: 50, 216: 150}[p]
    current = torch.tensor([0, 1, 72, 80, 30])
    count = 24 + total
    mask = ref.quota_mask(risk, own, current, total)
    ids = ref.lut(risk, mask, own, count)
    for hh in range(h):
        a = int(current[hh])
        for tt in range(t):
            o = int(own[hh, tt])
            r = risk[hh, tt].clone()
            if p == 72:
                if o >= 24:
                    r[o] = torch.inf
                picked = _brute_top(r, range(24, 72), total)
            else:
                if p - 72 <= o:
                    r[o] = torch.inf
                picked = (_brute_top(r, range(p - 72, p), a) if a > 0 else []) + \
                    (_brute_top(risk[hh, tt], range(24, p - 72), total - a) if total - a > 0 else [])
            listed = set(range(24)) | set(picked)
            assert [i for i in range(p) if mask[hh, tt, i]] == sorted(listed)
            entries = [o] + _brute_top(risk[hh, tt], sorted(listed - {o}), len(listed))
            want = (entries + [-1] * count)[:count]
            assert ids[hh, tt].tolist() == want, (p, hh, tt)


def test_selected_attention_skips_padding():
    """LUT entries outside [0, P) are not read: a table with -1 and
    out-of-window entries gives the output of the table without them."""
    g = torch.Generator().manual_seed(21)
    h, p, n = 2, 12, 128
    q = torch.randn(1, n, h, 128, generator=g).bfloat16()
    k = torch.randn(1, 64 * p, h, 128, generator=g).bfloat16()
    v = torch.randn(1, 64 * p, h, 128, generator=g).bfloat16()
    kp = k[0].transpose(0, 1).reshape(h, p, 64, 128)
    vp = v[0].transpose(0, 1).reshape(h, p, 64, 128)
    basis = workload.pca_basis(vp.float())
    s = workload.kmeans_summaries(kp, vp, basis, torch.Generator().manual_seed(3))
    ids = torch.tensor([[[11, 2, 5], [10, 0, 7]]] * h).int()
    padded = torch.tensor([[[11, -1, 2, p, 5, -1], [10, 0, -1, 7, 99, -1]]] * h).int()
    want = ref.selected_attention(q, k, v, s, basis, ids, dtype=torch.float64)
    got = ref.selected_attention(q, k, v, s, basis, padded, dtype=torch.float64)
    torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-12)
    assert torch.equal(ref.mask_from_ids(padded, p), ref.mask_from_ids(ids, p))


def test_select_topk_semantics():
    p = 216
    risk = _adversarial_rows(p, 6, 13).reshape(2, 3, p)
    own = torch.tensor([[150, 151, 152], [200, 201, 202]])
    ids, mask = ref.select_topk(risk, own, p // 10)
    for hh in range(2):
        for tt in range(3):
            cand = [i for i in range(p) if i != own[hh, tt]]
            assert ids[hh, tt].tolist() == [int(own[hh, tt])] + _brute_top(risk[hh, tt], cand, p // 10 - 1)
            assert int(mask[hh, tt].sum()) == p // 10


def test_near_tie_order_rows():
    """Consecutive ranked pages within 1e-3 relative flag the row; the
    unranked prefix (own + anchors) is ignored."""
    r = torch.tensor([[[5.0, 4.0, 3.0, 2.0, 1.0], [5.0, 4.0, 3.0, 2.9995, 1.0]]])
    ids = torch.tensor([[[0, 1, 2, 3, 4], [0, 1, 2, 3, 4]]])
    assert ref.near_tie_order_rows(r, ids, 1).tolist() == [[False, True]]
    r2 = torch.tensor([[[5.0, 4.9999, 3.0, 2.0, 1.0]]])
    assert ref.near_tie_order_rows(r2, ids[:, :1], 2).tolist() == [[False]]
    assert ref.near_tie_order_rows(r2, ids[:, :1], 0).tolist() == [[True]]


def test_near_tie_rows():
    r = torch.tensor([[[5.0, 4.0, 3.9999, 1.0], [5.0, 4.0, 3.0, 1.0]]])
    ties = ref.near_tie_rows(r, torch.tensor([[2, 2]]))
    assert ties.tolist() == [[True, False]]


def test_kmeans_summary_contract():
    """Summary invariants of the synthetic inputs: reps re-centred on the page
    key mean (RV/ops.py:60), mean = bf16(V mean), page scalar slots
    (RV/ops.py:74-75), zero reserved slots, Haar rows zero-sum."""
    h, p = 2, 5
    g = torch.Generator().manual_seed(1)
    k = torch.randn(h, p, 64, 128, generator=g).bfloat16()
    v = torch.randn(h, p, 64, 128, generator=g).bfloat16()
    basis = workload.pca_basis(v.float())
    s = workload.kmeans_summaries(k, v, basis, torch.Generator().manual_seed(2))
    assert s.keys.shape == (h, p, 4, 128) and s.detail.shape == (h, p, 3, 8) and s.stats.shape == (h, p, 4, 12)
    assert s.bytes() == h * p * 1424
    torch.testing.assert_close(s.keys.float().mean(2), k.float().mean(2), atol=2e-2, rtol=0)
    assert torch.equal(s.mean, v.float().mean(2).bfloat16())
    torch.testing.assert_close(s.stats[:, :, 1, 11].float(), v.float().norm(dim=-1).amax(2), atol=0, rtol=8e-3)
    assert (s.stats[:, :, 2:, 11] == 0).all()
    torch.testing.assert_close(basis.transpose(1, 2) @ basis, torch.eye(8).expand(h, 8, 8), atol=1e-5, rtol=0)
    assert torch.equal(torch.tensor(ref.HAAR).sum(1), torch.zeros(3, dtype=torch.int64))


def test_quota_table_contract():
    tab = workload.quota_table(2)
    a, b = tab[..., 0], tab[..., 1]
    assert (a >= 4).all() and (a <= 36).all() and (b >= 0).all() and (b <= 40).all()
    n = a + b
    assert (n == n[..., :1]).all()
    assert abs(float(n.float().mean()) - 40.8) < 1.5


def test_select_counts_reference_contract():
    """The reference's own CPU contract for RouteOps.select
    (RV/test_ops.py:39-47): every page eligible at threshold -1 on a 410-page
    window caps the count at ceil(0.25 * 410) = 103 with 307 overflow, own is
    selected, ids past the count are -1, the mask holds count pages."""
    g = torch.Generator().manual_seed(192)
    scores = torch.rand(2, 3, 410, generator=g)
    own = torch.tensor([[338, 339, 340]]).expand(2, -1)
    s = ref.select_counts(scores, own, threshold=-1)
    assert (s['counts'] == 103).all() and (s['overflow'] == 307).all()
    assert s['mask'].gather(-1, own[..., None]).all()
    assert (s['ids'][..., 103:] == -1).all() and s['ids'].shape[-1] == 128
    assert (s['mask'].sum(-1) == s['counts']).all()


def _brute_select(sc, own, valid, threshold, density, max_fraction, cap_ids):
    """Plain-Python RouteOps.select of one row."""
    p = len(sc)
    cap = min(cap_ids, math.ceil(max_fraction * p))
    key = lambda i: (2, 0.0) if i == own else ((1, sc[i]) if valid[i] else (0, 0.0))
    order = sorted(range(p), key=lambda i: (key(i)[0], key(i)[1], -i), reverse=True)
    if threshold is None:
        count, over = min(max(1, math.floor(p * density)), sum(valid)), 0
    else:
        wanted = sum(1 for i in range(p) if (valid[i] and sc[i] > threshold) or i == own)
        count, over = min(max(wanted, 1), cap), max(wanted - cap, 0)
    chosen = order[:count]
    resid = sum(sc[i] for i in range(p) if valid[i] and i not in chosen)
    return chosen, count, over, resid


@pytest.mark.parametrize("threshold", [None, 0.0, 3.5, 100.0])
def test_select_counts_brute_force(threshold):
    """Integer-binned scores (many ties), a random valid mask with own valid,
    thresholds below, inside and above the score range: ids, counts, overflow,
    mask and residual risk equal a plain-Python restatement."""
    g = torch.Generator().manual_seed(7)
    h, t, p = 2, 3, 96
    scores = torch.randint(-3, 8, (h, t, p), generator=g).float()
    valid = torch.rand(h, t, p, generator=g) > 0.2
    own = torch.randint(0, p, (h, t), generator=g)
    valid.scatter_(-1, own[..., None], True)
    s = ref.select_counts(scores, own, threshold=threshold, valid=valid, density=0.1, max_fraction=0.25,
                          id_capacity=40)
    for hh in range(h):
        for tt in range(t):
            chosen, count, over, resid = _brute_select(scores[hh, tt].tolist(), int(own[hh, tt]),
                                                      valid[hh, tt].tolist(), threshold, 0.1, 0.25, 40)
            assert int(s['counts'][hh, tt]) == count and int(s['overflow'][hh, tt]) == over
            assert s['ids'][hh, tt].tolist() == chosen + [-1] * (40 - count)
            assert sorted(torch.nonzero(s['mask'][hh, tt]).flatten().tolist()) == sorted(chosen)
            assert float(s['residual_risk'][hh, tt]) == resid
