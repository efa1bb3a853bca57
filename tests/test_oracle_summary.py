"""Pins the summary oracle (oracle/summary.py): k-means against a plain-Python
Lloyd loop, cluster-structured pages against their closed form, and the
summary contract's scalar slots against direct definitions."""
import math

import torch

from oracle import summary as osum
from streaming_sparse_amd import workload


def _py_lloyd(k, init, iters=4):
    """Lloyd iterations in plain Python floats on one page."""
    pts = [[float(x) for x in row] for row in k.tolist()]
    cent = [list(pts[i]) for i in init]
    assign = None
    for _ in range(iters):
        assign = []
        for pnt in pts:
            dists = [sum((a - b) ** 2 for a, b in zip(pnt, c)) for c in cent]
            assign.append(min(range(4), key=lambda r: (dists[r], r)))
        for r in range(4):
            mem = [pts[t] for t in range(len(pts)) if assign[t] == r]
            if mem:
                cent[r] = [sum(col) / len(mem) for col in zip(*mem)]
    return cent, assign


def test_kmeans_matches_python_loop():
    g = torch.Generator().manual_seed(3)
    k = torch.randn(2, 64, 128, generator=g).bfloat16().float()
    init = torch.tensor([[0, 5, 17, 40], [63, 2, 31, 9]])
    cent, assign, margin = osum.kmeans(k, init)
    for b in range(2):
        pc, pa = _py_lloyd(k[b], init[b].tolist())
        assert assign[b].tolist() == pa
        torch.testing.assert_close(cent[b], torch.tensor(pc), atol=1e-5, rtol=1e-5)
    assert (margin > 0).all()


def test_separated_clusters_closed_form():
    """4 tight clusters of 16 tokens around distant centres, init one token
    from each: the assignment is the planted partition, reps re-centre the
    cluster means, and the variance / spread slots are the planted ones."""
    g = torch.Generator().manual_seed(7)
    centers = torch.randn(4, 128, generator=g) * 10
    noise = torch.randn(64, 128, generator=g) * 0.01
    label = torch.arange(64) % 4
    k = (centers[label] + noise).bfloat16()
    v = torch.randn(64, 128, generator=g).bfloat16()
    init = torch.tensor([[[0, 1, 2, 3]]])
    basis = workload.pca_basis(v.float()[None, None])
    out = osum.summaries(k[None, None], v[None, None], basis, init)
    kf, vf = k.float(), v.float()
    km = torch.stack([kf[label == r].mean(0) for r in range(4)])
    pk = (km - km.mean(0) + kf.mean(0)).bfloat16()
    assert torch.equal(out['keys'][0, 0], pk)
    vm = torch.stack([vf[label == r].mean(0) for r in range(4)])
    spread = torch.stack([((vf[label == r] - vm[r]) ** 2).sum(-1).mean().sqrt() for r in range(4)])
    torch.testing.assert_close(out['stats'][0, 0, :, 10].float(), spread, atol=0, rtol=8e-3)
    var = torch.stack([((kf[label == r] - km[r]) ** 2).mean(0) for r in range(4)])
    torch.testing.assert_close(out['stats'][0, 0, :, :8].float(), var.reshape(4, 8, 16).mean(-1), atol=1e-7,
                               rtol=8e-3)
    assert torch.equal(out['mean'][0, 0], vf.mean(0).bfloat16())
    torch.testing.assert_close(out['stats'][0, 0, 1, 11].float(), vf.norm(dim=-1).amax(), atol=0, rtol=8e-3)
    assert (out['stats'][0, 0, 2:, 11] == 0).all()


def test_identical_keys_collapse():
    """All keys equal: every distance ties, all tokens join cluster 0, the
    other clusters stay empty at their (identical) initial centroids; the
    empty clusters take the page V mean, so their detail contrasts vanish
    against cluster 0 only through the V means."""
    g = torch.Generator().manual_seed(1)
    k = torch.randn(1, 128, generator=g).expand(64, 128).bfloat16()
    v = torch.randn(64, 128, generator=g).bfloat16()
    cent, assign, _ = osum.kmeans(k.float()[None], torch.tensor([[0, 1, 2, 3]]))
    assert (assign == 0).all()
    out = osum.summaries(k[None, None], v[None, None], torch.eye(128, 8)[None], torch.tensor([[[0, 1, 2, 3]]]))
    # every cluster V mean equals the page V mean -> all Haar contrasts are 0
    assert (out['detail'] == 0).all()
    assert (out['stats'][0, 0, :, :8] == 0).all()


def test_oracle_matches_input_generator():
    """The synthetic inputs' summaries (streaming_sparse_amd.workload) are the
    same function: identical bf16 outputs for the same initial tokens except
    pages whose k-means has a near tie."""
    g = torch.Generator().manual_seed(11)
    h, p = 2, 12
    k = torch.randn(h, p, 64, 128, generator=g).bfloat16()
    v = torch.randn(h, p, 64, 128, generator=g).bfloat16()
    basis = workload.pca_basis(v.float())
    init = workload.kmeans_init(h, p, torch.Generator().manual_seed(5))
    want = workload.kmeans_summaries(k, v, basis, init)
    got = osum.summaries(k, v, basis, init)
    ok = got['margin'] > 1e-5
    for name in ('keys', 'mean', 'detail', 'stats'):
        a = getattr(want, name).float()[ok]
        b = got[name].float()[ok]
        assert bool(((a - b).abs() <= b.abs() * 2.0 ** -7 + 1e-6).all()), name
    assert int(ok.sum()) >= h * p - 1
