"""Current-chunk summary recompute on the HIP path vs. the oracle
(oracle/summary.py) on identical seeded inputs: the 72 current pages x 12
heads of a 432-page window, written into the window's summary slab.

Bar: outputs bit-exact except one-ulp bf16 roundings (fp32 accumulation
order), on every page whose k-means has no near tie (best and second-best
centroid distance within 1e-5 relative in some iteration)."""
import pytest
import torch

from oracle import summary as osum
from streaming_sparse_amd import summary, workload
from streaming_sparse_amd.ops import Summary

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("iters", [4, 1, 2, 6])
def test_current_chunk_summaries_match_oracle(device, iters):
    """The kernel ends its Lloyd loop at the first assignment that repeats
    the previous one; the oracle runs every iteration.  1 iteration never
    reaches that exit, 6 reach it on nearly every page."""
    x = workload.make_call(cfg=3, frames=18)
    P = x.pages
    g = x.to(device)
    init = workload.kmeans_init(12, 72, torch.Generator().manual_seed(workload.seed_for(3, 1, 0, 9)))
    slab = Summary(*(getattr(g.summary, f).clone() for f in Summary.FIELDS))
    for f in Summary.FIELDS:
        getattr(slab, f)[:, P - 72:].zero_()
    summary.build(g.k, g.v, g.basis, init.to(device), slab, P - 72, 72, iters=iters)
    torch.cuda.synchronize()
    kp = x.k[0].transpose(0, 1).reshape(12, P, 64, 128)[:, P - 72:]
    vp = x.v[0].transpose(0, 1).reshape(12, P, 64, 128)[:, P - 72:]
    want = osum.summaries(kp, vp, x.basis, init, iters=iters)
    ok = want['margin'] > 1e-5
    print(f"{int(ok.sum())}/{ok.numel()} pages without a k-means near tie", flush=True)
    assert int(ok.sum()) >= ok.numel() * 0.95
    for name in ('keys', 'mean', 'detail', 'stats'):
        got = getattr(slab, name)[:, P - 72:].cpu().float()[ok]
        ref = want[name].float()[ok]
        err = (got - ref).abs()
        bound = ref.abs() * 2.0 ** -7 + 1e-6
        diff = int((got != ref).sum())
        print(f"{name}: {diff} of {ref.numel()} values differ, max abs {float(err.max()):.2e}", flush=True)
        assert bool((err <= bound).all()), name
        assert diff <= ref.numel() * 1e-3, name
    # pages outside the range are untouched
    for f in Summary.FIELDS:
        assert torch.equal(getattr(slab, f)[:, :P - 72].cpu(), getattr(x.summary, f)[:, :P - 72])


def test_summary_write_through_equals_copy_then_summary(device):
    """ssa_summary_write: the chunk's K/V written into the cache pages in the
    pass that summarises them gives the cache and the summaries of a copy
    followed by ssa_summary, bit for bit; pages outside the range stay as
    they were.  Sources: a fresh [4608, H, 128] chunk and a strided view
    (every other token row of a larger buffer)."""
    x = workload.make_call(cfg=3, frames=18)
    P = x.pages
    g = x.to(device)
    init = workload.kmeans_init(12, 72, torch.Generator().manual_seed(11)).to(device)
    gen = torch.Generator(device=device).manual_seed(5)
    big_k = torch.randn(2 * 4608, 12, 128, generator=gen, device=device).to(torch.bfloat16)
    big_v = torch.randn(2 * 4608, 12, 128, generator=gen, device=device).to(torch.bfloat16)
    for name, sk, sv in (("contiguous", big_k[:4608], big_v[:4608]), ("strided", big_k[::2], big_v[::2])):
        outs = []
        for fused in (False, True):
            k, v = g.k.clone(), g.v.clone()
            slab = Summary(*(getattr(g.summary, f).clone() for f in Summary.FIELDS))
            if fused:
                summary.build(k, v, g.basis, init, slab, P - 72, 72, src=(sk, sv))
            else:
                k[0, 64 * (P - 72):].copy_(sk)
                v[0, 64 * (P - 72):].copy_(sv)
                summary.build(k, v, g.basis, init, slab, P - 72, 72)
            outs.append((k, v, slab))
        torch.cuda.synchronize()
        (k0, v0, s0), (k1, v1, s1) = outs
        same_kv = torch.equal(k0.view(torch.int16), k1.view(torch.int16)) and \
            torch.equal(v0.view(torch.int16), v1.view(torch.int16))
        same_s = all(torch.equal(getattr(s0, f).view(torch.int16), getattr(s1, f).view(torch.int16))
                     for f in Summary.FIELDS)
        print(f"{name}: cache equal {same_kv}, summaries equal {same_s}", flush=True)
        assert same_kv and same_s
        assert torch.equal(k1[0, :64 * (P - 72)].view(torch.int16), g.k[0, :64 * (P - 72)].view(torch.int16))
