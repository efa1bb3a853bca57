"""One call of the hot path (the base-tier route with rep values on the
side, then the fused attention, two-term P.V) captured in a HIP graph and
replayed: the library allocates nothing, never synchronises and works on the
caller's stream, so the captured launches replay it.  Three replays, with
eager work of the program and a synchronisation between them, each give the
eager call's output and page table bit for bit (216-page window, 12 heads x
4608 queries)."""
import pytest
import torch

from streaming_sparse_amd import workload
from streaming_sparse_amd.attention import Workspace
from streaming_sparse_amd.legacy_components import attention
from streaming_sparse_amd.route import route

pytestmark = pytest.mark.gpu


def test_call_replays_in_a_graph(device):
    g = workload.make_call(cfg=0, frames=9).to(device)
    P, H, D = g.pages, 12, 128
    ws = Workspace()
    basis = g.basis.to(torch.bfloat16).contiguous()
    ops = ws.tensor('graph_rep_ops', (H, (P + 15) // 16, 512), device, torch.bfloat16)

    def call():
        ids, _, _, _ = route(g.q, g.summary, g.theta, tier='base', workspace=ws, want_mask=False, rep_out=ops)
        return ids, attention(g.q, g.k, g.v, g.summary, basis, ids, ws, rep_ops=ops)

    ids, out = call()                      # eager: also creates every workspace buffer
    torch.cuda.synchronize()
    want_ids, want_out = ids.clone(), out.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()                             # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gids, gout = call()
    for r in range(3):
        gout.zero_()
        gids.fill_(-7)
        junk = torch.randn(1 << 20, device=device).sum()   # the program's own eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        same_ids = torch.equal(gids, want_ids)
        same_out = torch.equal(gout.view(torch.int16), want_out.view(torch.int16))
        print(f"replay {r}: ids equal {same_ids}, output equal {same_out} ({float(junk):.1f})", flush=True)
        assert same_ids and same_out
