"""The grouping oracle (oracle/group.py) pinned without the reference:
closed forms of special cases and invariants.

* Features varying along one dimension only: every level's direction stays
  that axis, so the whole balanced order is one stable argsort of it.
* A dominant principal axis with gaps at the split quantiles: the first
  split is by the projection on the top eigenvector of the covariance
  (numpy eigh), sign fixed by the highest-variance axis the iteration
  starts from.
* gate = 0: features are the centred key projections scaled to unit RMS
  (zero token mean per feature, unit RMS); bank = 0: the softmax is uniform
  and features are 0.1 tanh(gate) times the unit-RMS centred value
  projections.
* Token permutation equivariance of the features; permutations out; the
  first chunk's frame re-sort puts the anchor frame in pages 0..23.
"""
import numpy as np
import torch

from oracle import group as og


def test_balanced_one_axis_is_a_global_sort():
    g = torch.Generator().manual_seed(1)
    h, n, d = 2, 4608, 32
    x = torch.zeros(h, n, d, dtype=torch.float64)
    x[..., 5] = torch.randn(h, n, generator=g, dtype=torch.float64)
    x[..., 9] = 3.0                                   # a constant dimension changes nothing
    ids = og.balanced(x, og.SPLITS + og.INNER)
    want = x[..., 5].argsort(dim=-1, stable=True)
    assert torch.equal(ids, want)


def test_balanced_first_split_follows_top_eigenvector():
    rng = np.random.default_rng(2)
    n, d = 4608, 32
    u = rng.normal(size=d)
    u /= np.linalg.norm(u)
    z = rng.normal(size=n)
    z = np.sort(z)
    z[n // 3:] += 5.0                                 # gaps at both split quantiles
    z[2 * n // 3:] += 5.0
    z = rng.permutation(z)
    x = 10.0 * z[:, None] * u[None, :] + 0.01 * rng.normal(size=(n, d))
    ids = og.balanced(torch.tensor(x)[None], (3,))[0].numpy()
    xc = x - x.mean(0)
    w, vec = np.linalg.eigh(xc.T @ xc)
    top = vec[:, -1]
    start = np.argmax((xc ** 2).mean(0))
    top = top * np.sign(top[start])
    proj = xc @ top
    want = np.argsort(proj, kind="stable")
    for part in range(3):
        sl = slice(part * n // 3, (part + 1) * n // 3)
        assert set(ids[sl].tolist()) == set(want[sl].tolist())


def _inputs(seed, h=2, t=4608, d=128, r=32):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(h, t, d, generator=g).bfloat16()
    v = torch.randn(h, t, d, generator=g).bfloat16()
    bank = torch.randn(h, r, d, generator=g)
    gv = torch.nn.functional.normalize(bank, dim=-1).transpose(1, 2).contiguous()
    gate = 0.1 + 0.05 * torch.randn(h, r, generator=g)
    return k, v, bank, gv, gate


def test_features_gate_zero_and_bank_zero():
    k, v, bank, gv, gate = _inputs(3)
    f = og.group_features(k, v, bank, gv, torch.zeros_like(gate))
    torch.testing.assert_close(f.mean(1), torch.zeros_like(f.mean(1)), atol=1e-12, rtol=0)
    torch.testing.assert_close(f.square().mean((1, 2)), torch.ones(2, dtype=torch.float64), atol=1e-12, rtol=0)
    f0 = og.group_features(k, v, torch.zeros_like(bank), gv, gate)
    resp = f0 / (0.1 * gate.double().tanh())[:, None, :]
    vp = torch.einsum('htd,hdr->htr', v.double(), gv.double())
    want = vp - vp.mean(1, keepdim=True)
    want = want / want.square().mean((1, 2), keepdim=True).sqrt()
    torch.testing.assert_close(resp, want, atol=1e-10, rtol=1e-10)


def test_features_token_equivariance_and_orders_are_permutations():
    k, v, bank, gv, gate = _inputs(4)
    perm = torch.randperm(4608, generator=torch.Generator().manual_seed(5))
    f = og.group_features(k, v, bank, gv, gate)
    fp = og.group_features(k[:, perm], v[:, perm], bank, gv, gate)
    torch.testing.assert_close(fp, f[:, perm], atol=1e-12, rtol=1e-12)
    order = og.group_order(k, v, bank, gv, gate)
    assert torch.equal(order.sort(-1).values, torch.arange(4608).expand(2, -1))
    first = og.group_order(k, v, bank, gv, gate, first_chunk=True)
    assert bool((first[:, :1536] < 1536).all()) and bool((first[:, 3072:] >= 3072).all())
    # the frame re-sort keeps the grouped order within each frame
    for h in range(2):
        in_frame0 = [int(t) for t in order[h] if t < 1536]
        assert first[h, :1536].tolist() == in_frame0


def test_page_order():
    assert torch.equal(og.page_order(360), torch.arange(72))
    po = og.page_order(338)
    assert po[:22].tolist() == [0, 3, 6, 9, 13, 16, 19, 22, 26, 29, 32, 36, 39, 42, 45, 49, 52, 55, 58, 62, 65, 68]
    assert sorted(po.tolist()) == list(range(72))
