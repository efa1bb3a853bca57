"""RouteOps.select on the HIP path (ssa_select) against the oracle
(oracle/reference.py select_counts) on identical inputs: the reference's own
contract case (RV/test_ops.py:39-47: 410 pages, threshold -1), integer-binned
scores full of ties with a valid mask and thresholds below, inside and above
the score range, and the 432-page window at 12 heads x 72 blocks with float
scores in both count modes.  ids, counts, mask and overflow must be equal;
the residual risk (a float32 sum in another order) within 1e-5 relative."""
import pytest
import torch

from oracle import reference as ref
from streaming_sparse_amd.route import select

pytestmark = pytest.mark.gpu


def _check(got, want, tag):
    for name in ("ids", "counts", "overflow"):
        assert torch.equal(got[name].cpu().long(), want[name].long()), (tag, name)
    assert torch.equal(got["mask"].cpu(), want["mask"]), (tag, "mask")
    r, w = got["residual_risk"].cpu().double(), want["residual_risk"]
    err = float(((r - w).abs() / w.abs().clamp_min(1.0)).max())
    print(f"{tag}: counts {got['counts'].cpu().unique().tolist()[:6]}, residual rel {err:.2e}", flush=True)
    assert err <= 1e-5, tag


def test_select_reference_contract(device):
    g = torch.Generator().manual_seed(192)
    scores = torch.rand(2, 3, 410, generator=g)
    own = torch.tensor([[338, 339, 340]]).expand(2, -1)
    got = select(scores.to(device), own.to(device), threshold=-1)
    assert (got["counts"] == 103).all() and (got["overflow"] == 307).all()
    assert (got["ids"][..., 103:] == -1).all()
    _check(got, ref.select_counts(scores, own, threshold=-1), "contract")


@pytest.mark.parametrize("threshold", [None, 0.0, 3.5, 100.0])
def test_select_ties_and_valid(device, threshold):
    g = torch.Generator().manual_seed(11)
    h, t, p = 3, 5, 96
    scores = torch.randint(-3, 8, (h, t, p), generator=g).float()
    scores[0, 0, :8] = -0.0            # signed zeros tie with +0.0
    valid = torch.rand(h, t, p, generator=g) > 0.2
    own = torch.randint(0, p, (h, t), generator=g)
    valid.scatter_(-1, own[..., None], True)
    kw = dict(threshold=threshold, valid=valid, density=0.1, max_fraction=0.25, id_capacity=40)
    got = select(scores.to(device), own.to(device), **{**kw, "valid": valid.to(device)})
    _check(got, ref.select_counts(scores, own, **kw), f"ties threshold={threshold}")


@pytest.mark.parametrize("threshold", [None, 0.9])
def test_select_full_window(device, threshold):
    g = torch.Generator().manual_seed(5)
    h, t, p = 12, 72, 432
    scores = torch.rand(h, t, p, generator=g) ** 3
    own = (p - 72 + torch.arange(t)).expand(h, t)
    got = select(scores.to(device), own.to(device), threshold=threshold)
    _check(got, ref.select_counts(scores, own, threshold=threshold), f"432 pages threshold={threshold}")
