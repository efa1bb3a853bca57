"""Clean-commit token grouping on the GPU (ssa_group_order) against the
float64 oracle (oracle/group.py) on identical seeded inputs: two layers x 12
heads batched in one call, the plain order, the first chunk's frame re-sort
and a non-identity page order.  Both run in float64, so the orders must agree
token for token."""
import pytest
import torch

from oracle import group as og
from streaming_sparse_amd import group, workload

pytestmark = pytest.mark.gpu


def inputs(seed, layers=2, heads=12):
    g = torch.Generator().manual_seed(workload.seed_for(4, 0, 0, 40 + seed))
    k = torch.randn(layers, 4608, heads, 128, generator=g)
    v = torch.randn(layers, 4608, heads, 128, generator=g)
    freqs = workload.rope_table(128)
    k = torch.stack([workload.apply_rope(k[l], 3, freqs) for l in range(layers)])
    return k.bfloat16(), v.bfloat16()


@pytest.mark.parametrize("first_chunk,history", [(False, 360), (True, 360), (False, 338)])
def test_group_order_matches_oracle(device, first_chunk, history):
    k, v = inputs(0)
    w = group.GroupWeights.seeded(2, 12, 5, device)
    pd = group.page_destinations(history)
    got = group.order(k.to(device), v.to(device), w, first_chunk=first_chunk, page_dst=pd).cpu()
    pages = og.page_order(history)
    for layer in range(2):
        want = og.group_order(k[layer].transpose(0, 1), v[layer].transpose(0, 1), w.bank[layer].cpu(),
                              w.group_v[layer].cpu(), w.gate[layer].cpu(), pages=pages, first_chunk=first_chunk)
        same = (got[layer] == want).all(-1)
        print(f"layer {layer} first_chunk={first_chunk} history={history}: {int(same.sum())}/12 heads identical",
              flush=True)
        assert torch.equal(got[layer].long(), want)
