"""The route boundary in the reference's call shape: graph.BatchGraphs
(VB/graph.py:59-93 get, :212-221 replay) over ssa_route / ssa_pset.

A captured entry replays, with the program's own eager work and a
synchronisation between replays, the same (ids, mask, risk, stats) as the
eager route(...) bit for bit: the intersection tier with Full_Pset on heads
{3, 4, 9} at 432 pages, a second query batch and own table copied in by
replay, quotas changed in place between replays (as queue_policy.attach does,
VB/queue_policy.py:25-33), and the base tier fed the probe rows themselves
([H, T, 16, D], the reference's input_m16 mode).  The entry's operand tiles
drive the attention call that follows, bit for bit as route's."""
import pytest
import torch

from streaming_sparse_amd import pset, workload
from streaming_sparse_amd.attention import Workspace
from streaming_sparse_amd.graph import BatchGraphs
from streaming_sparse_amd.legacy_components import attention
from streaming_sparse_amd.route import route

pytestmark = pytest.mark.gpu
HEADS = [3, 4, 9]
PROBE_ROWS = [(42 * m + 5) // 10 for m in range(16)]     # round(63 m / 15)


def blocks(q):
    """[1, N, H, D] queries -> the reference's [H, T, 64, D] blocks."""
    _, n, h, d = q.shape
    return q[0].reshape(n // 64, 64, h, d).permute(2, 0, 1, 3).contiguous()


def same(a, b):
    return torch.equal(a.view(torch.int32) if a.dtype == torch.float32 else a,
                       b.view(torch.int32) if b.dtype == torch.float32 else b)


def test_replay_equals_route_intersection_full_pset(device):
    x = workload.make_call(cfg=3, frames=18)
    g = x.to(device)
    reader = pset.Reader(workload.reader_weights(), device)
    enc = pset.encode(g.summary, g.basis, reader)
    tab = workload.quota_table(3)
    a = tab[0, 3, :, 0].to(device)
    n = int(tab[0, 3, 0].sum())
    bg = BatchGraphs('intersection', reader=reader)
    bg.n = n
    bg.current_slots = a.clone()
    e = bg.get(blocks(g.q), g.summary, enc, g.theta, g.basis, g.own, True, torch.tensor(HEADS))
    assert e['graph'] is not None

    def eager(q, cur):
        out = route(q, g.summary, g.theta, tier='intersection', own=g.own, current_slots=cur, n=n,
                    workspace=Workspace(), full_pset=HEADS, encoding=enc, reader=reader)
        return [t.clone() for t in out]

    x2 = workload.make_call(cfg=3, frames=18, layer=2)
    q2 = x2.q.to(device)
    cases = [("first batch", g.q, a), ("second batch", q2, a), ("quotas changed in place", q2, a.flip(0))]
    for name, q, cur in cases:
        want = eager(q, cur)
        bg.current_slots.copy_(cur)
        qb = blocks(q)
        for r in range(2):
            e['ids'].fill_(-7)
            e['risk'].zero_()
            junk = torch.randn(1 << 20, device=device).sum()     # the program's own eager work
            got = bg.replay(e, qb, g.own)
            torch.cuda.synchronize()
            ok = [same(x_, y_) for x_, y_ in zip(got, want)]
            print(f"{name}, replay {r}: ids/mask/risk/stats equal {ok}, executed {int(got[3][0])} "
                  f"({float(junk):.1f})", flush=True)
            assert all(ok)
    # the attention call after the graph takes the entry's operand tiles
    ws = Workspace()
    want_ids = eager(q2, a.flip(0))[0]
    o1 = attention(q2, g.k, g.v, g.summary, g.basis, e['ids'], ws, rep_ops=e['rep_ops']).clone()
    o2 = attention(q2, g.k, g.v, g.summary, g.basis, want_ids, ws).clone()
    torch.cuda.synchronize()
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16))
    assert bg.calls == 6 and len(bg.entries) == 1


def test_replay_equals_route_base_probe_rows(device):
    g = workload.make_call(cfg=0, frames=9).to(device)
    bg = BatchGraphs('base')
    probes = blocks(g.q)[:, :, PROBE_ROWS].contiguous()       # [H, T, 16, D]
    e = bg.get(probes, g.summary, None, g.theta, g.basis, g.own, False)
    want = [t.clone() for t in route(g.q, g.summary, g.theta, tier='base', own=g.own, workspace=Workspace())]
    for r in range(3):
        e['ids'].fill_(-7)
        junk = torch.randn(1 << 20, device=device).sum()
        got = bg.replay(e, probes, g.own)
        torch.cuda.synchronize()
        ok = [same(x_, y_) for x_, y_ in zip(got, want)]
        print(f"base probe rows, replay {r}: equal {ok} ({float(junk):.1f})", flush=True)
        assert all(ok)


def test_near_tie_report_replays_in_a_graph(device):
    """The near-tie report's counter is zeroed by a launch of the call
    itself, so a captured route replays the same count and rows."""
    g = workload.make_call(cfg=0, frames=9).to(device)
    rows = torch.full((12 * 72,), -1, dtype=torch.int32, device=device)
    cnt = torch.zeros(1, dtype=torch.int32, device=device)
    ws = Workspace()
    call = lambda: route(g.q, g.summary, g.theta, tier='base', own=g.own, workspace=ws, ties=(rows, cnt),
                         tie_eps=1e-3)
    call()
    torch.cuda.synchronize()
    want_k = int(cnt.item())
    want = rows[:want_k].sort().values.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    for r in range(3):
        cnt.fill_(999)
        rows.fill_(-1)
        junk = torch.randn(1 << 20, device=device).sum()
        graph.replay()
        torch.cuda.synchronize()
        k = int(cnt.item())
        print(f"replay {r}: {k} near-tie rows (eager {want_k}) ({float(junk):.1f})", flush=True)
        assert k == want_k and torch.equal(rows[:k].sort().values, want)
