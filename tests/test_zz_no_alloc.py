"""The allocation-free Full_Pset entry point (ssa_pset_noalloc, scratch in the
library's own device array) against the entry point with caller-owned
scratch (ssa_pset), through the C ABI on identical inputs: two calls in a row,
the second with a smaller input (fewer scoped heads, a smaller window), so
the second reuses scratch the first left behind.  The kernels are the same and
their only atomics count integers, so every output must agree bit for bit:
the corrected mask and page table, the per-row gains, decisions and scores,
and the three counters."""
import pytest
import torch

from streaming_sparse_amd import _lib, pset, workload
from streaming_sparse_amd.attention import Workspace
from streaming_sparse_amd.route import route

pytestmark = pytest.mark.gpu


def routed(device, frames, heads):
    x = workload.make_call(cfg=3, frames=frames)
    g = x.to(device)
    reader = pset.Reader(workload.reader_weights(), device)
    enc = pset.encode(g.summary, g.basis, reader)
    tab = workload.quota_table(3)
    a, n = tab[0, 3, :, 0], int(tab[0, 3, 0].sum())
    lse = torch.empty(12, 72, 16, device=device)
    ids, mask, risk, _ = route(g.q, g.summary, g.theta, tier='intersection', own=g.own, current_slots=a, n=n,
                               workspace=Workspace(), lse_out=lse)
    return g, reader, enc, ids, mask, risk, lse, heads


def correct_both(case):
    g, reader, enc, ids, mask, risk, lse, heads = case
    out = {}
    for no_alloc in (False, True):
        m = mask.clone()
        i = ids.clone()
        stats, rows = pset.correct(g.q, g.summary, enc, reader, risk, lse, m, i, g.own, heads, want_scores=True,
                                   no_alloc=no_alloc)
        torch.cuda.synchronize()
        out[no_alloc] = dict(mask=m.cpu(), ids=i.cpu(), stats=stats.cpu().clone(), gain=rows['gain'].cpu().clone(),
                             executed=rows['executed'].cpu().clone(), argmax=rows['argmax'].cpu().clone(),
                             nonfinite=rows['nonfinite'].cpu().clone(), scores=rows['scores'].cpu().clone())
    return out[False], out[True]


def assert_same(a, b, tag):
    for k in a:
        x, y = a[k], b[k]
        if x.is_floating_point():
            same = torch.equal(x.view(torch.int64), y.view(torch.int64))
        else:
            same = torch.equal(x, y)
        assert same, (tag, k)
    print(f"{tag}: identical; executed {int(a['stats'][0])} of {int(a['stats'][1])} rows", flush=True)


def test_pset_noalloc_matches_caller_scratch(device):
    big = routed(device, 18, [3, 4, 9])          # 432 pages, 3 x 72 rows: the scratch limit
    a, b = correct_both(big)
    assert_same(a, b, "432 pages, heads 3,4,9")
    small = routed(device, 12, [4])              # 288 pages, 1 x 72 rows
    a, b = correct_both(small)
    assert_same(a, b, "288 pages, head 4")


def test_pset_noalloc_rejects_oversize(device):
    """More than 216 scoped rows is rejected before any launch."""
    g, reader, enc, ids, mask, risk, lse, _ = routed(device, 18, [0])
    with pytest.raises(RuntimeError):
        pset.correct(g.q, g.summary, enc, reader, risk, lse, mask.clone(), ids.clone(), g.own, [0, 1, 2, 3],
                     no_alloc=True)
