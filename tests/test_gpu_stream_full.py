"""The full streaming workload at its real size: 30 layers x 12 heads, 4
denoise steps + the clean step, a 360-page history ring (432-page window),
Full_Pset on layers {3,4,5,8,14,17,27} x heads {3,4,9} at step 0.  The
oracle would take hours over a whole chunk, so the whole chunk is checked
through size-independent properties and single calls against the oracle.

Two runtimes built from the same seed run chunks 0..6 (the window fills at
chunk 5; chunk 6 runs after the ring wrapped and the anchor was rebased):
* every call of chunk 6 (150 of them) gives bit-identical outputs in both,
  and so do their ring and summary state afterwards (no atomics or
  order-dependent reductions anywhere on the path);
* the call counts are the workload's: 116 sparse calls (7 with Full_Pset)
  and 34 dense ones per full-window chunk;
* every output is finite;
and, against the oracle, one Full_Pset call of chunk 7 (page table and
output), its first (dense) call and its commit grouping on three layers."""
import pytest
import torch

from streaming_sparse_amd.runtime import StreamConfig, StreamRuntime

pytestmark = pytest.mark.gpu


def run(device, chunks=7):
    rt = StreamRuntime(StreamConfig(seed=9), device)
    for c in range(chunks):
        before = dict(rt.calls)
        if c == chunks - 1:
            rt.record = []
        rt.run_chunk(rt.chunk_inputs())
        torch.cuda.synchronize()
        delta = {k: rt.calls[k] - before[k] for k in before}
        print(f"chunk {c}: history {rt.ring.n}, calls {delta}", flush=True)
    return rt, delta


def test_full_stream_repeat_and_counts(device):
    a, calls = run(device)
    assert calls == dict(sparse=116, dense=34, full_pset=7)
    assert a.calls_per_chunk() == calls
    outs_a = a.record
    assert len(outs_a) == 150
    assert all(bool(torch.isfinite(o.float()).all()) for o in outs_a)
    b, _ = run(device)
    same = [torch.equal(x.view(torch.int16), y.view(torch.int16)) for x, y in zip(outs_a, b.record)]
    print(f"{sum(same)}/150 calls bit-identical", flush=True)
    assert all(same)
    for la, lb in zip(a.layers, b.layers):
        assert torch.equal(la.k.view(torch.int16), lb.k.view(torch.int16))
        assert torch.equal(la.slab.keys.view(torch.int16), lb.slab.keys.view(torch.int16))
        assert torch.equal(la.slab.stats.view(torch.int16), lb.slab.stats.view(torch.int16))


def test_full_stream_call_matches_oracle(device):
    """One call of the full workload against the oracle: after chunks 0..6
    of the 30-layer runtime, chunk 7 (anchor rebased by 6 frames) step 0 of
    layer 4, an intersection call with Full_Pset on heads {3, 4, 9} over the
    full 432-page window.  Its page table equals the oracle chain (float64
    risk -> quota mask -> Full_Pset) on every row whose selection or swap
    decision is not a near tie, and its output matches
    SelectedAttention.fixed on its table (4 query blocks x 12 heads)."""
    import math

    from oracle import pset as opset
    from oracle import reference as ref
    from streaming_sparse_amd import workload
    from streaming_sparse_amd.ops import Summary
    from streaming_sparse_amd.runtime import CURRENT, PSET_HEADS

    rt, _ = run(device)
    inputs = rt.chunk_inputs()
    rt.begin_chunk()
    layer = 4
    q, k, v = inputs[0][layer]
    out = rt.layer_call(0, layer, q, k, v).clone()
    torch.cuda.synchronize()
    L = rt.layers[layer]
    P = rt.ring.n + CURRENT
    assert P == 432 and rt.calls['full_pset'] > 0
    ids = rt.last_ids.cpu()
    s = Summary(*(getattr(L.slab, f)[:, :P].cpu() for f in Summary.FIELDS))
    tiles = [0, 30, 50, 71]
    rows = torch.cat([torch.arange(t * 64, (t + 1) * 64) for t in tiles])
    want = ref.selected_attention(q.cpu(), L.k[:, :64 * P].cpu(), L.v[:, :64 * P].cpu(), s, L.basis.cpu().float(),
                                  ids, tiles=tiles).bfloat16()
    g, w_ = out[:, rows].cpu().float(), want[:, rows].float()
    err, mx = ref.rel_l2(g, w_), float((g - w_).abs().max())
    print(f"full-size call: rel-L2 {err:.3e} max-abs {mx:.3e}", flush=True)
    assert err <= 5e-3 and mx <= 2e-2
    # the page table against the oracle chain
    a_tab, n_tab = rt.quota(rt.chunk)
    a = a_tab[0, layer - 1].cpu().long()
    n = int(n_tab[0][layer - 1])
    own = (torch.arange(72) + P - 72)[None].expand(12, -1)
    pr = ref.probes(q.cpu())
    z = ref.route_logits(pr, s.keys)
    r64 = ref.risk(pr, ref.route_logits(pr, s.keys, torch.float64), s.stats, rt.theta.cpu(), dtype=torch.float64)
    m0 = ref.quota_mask(r64, own, a, n)
    enc = L.encoding
    enc_o = dict(co=enc.co[:, :P].cpu(), A=enc.A[:, :P].cpu(), mean=enc.mean[:, :P].cpu(),
                 detail=enc.detail[:, :P].cpu())
    w = workload.reader_weights(rt.cfg.seed)
    want_mask, orow, _ = opset.correct(pr.bfloat16().float(), z, r64.float(), m0, own, enc_o, w['wq'],
                                       list(PSET_HEADS))
    hist = r64.clone()
    hist[..., :24] = -math.inf
    hist[..., P - 72:] = -math.inf
    cur = r64.clone()
    cur[..., :P - 72] = -math.inf
    cur.scatter_(-1, own[..., None], math.inf)
    ties = ref.near_tie_rows(hist, (n - a)[:, None].expand_as(own)) | \
        ref.near_tie_rows(cur, a[:, None].expand_as(own))
    legal = orow['legal'].reshape(len(PSET_HEADS), 72, 16 * 32)
    scores = orow['scores'].flatten(-2)
    top = scores.masked_fill(~legal, -math.inf).topk(2, dim=-1).values
    scale = scores.masked_fill(~legal, 0).abs().amax(-1).clamp_min(1e-300)
    pset_ties = ((top[..., 0] - top[..., 1]).abs() <= 1e-3 * scale) | (top[..., 0].abs() <= 1e-3 * scale)
    ties[torch.tensor(PSET_HEADS)] |= pset_ties
    got_mask = ref.mask_from_ids(ids, P)
    same = (got_mask == want_mask).all(-1)
    print(f"full-size call: {int(same.sum())}/864 tables equal the oracle chain, {int(ties.sum())} near-tie rows",
          flush=True)
    assert bool((same | ties).all())


def test_full_stream_dense_call_and_commit_match_oracle(device):
    """The rest of a full-window chunk against the oracle: after chunks 0..6,
    chunk 7 runs whole.  Its first call (step 0, layer 0: dense, every one
    of the 432 pages exact, single-term P.V) matches dense attention over
    the window as the call saw it, on 4 query blocks x 12 heads; and its
    clean step's token grouping equals the float64 oracle's order token for
    token on three of the 30 layers (12 heads each; the first chunk's frame
    sort does not apply), with the ring's page order of a 360-page history."""
    from oracle import group as og
    from oracle import reference as ref
    from streaming_sparse_amd.runtime import CURRENT

    rt, _ = run(device)
    inputs = rt.chunk_inputs()
    rt.begin_chunk()
    P = rt.ring.n + CURRENT
    assert P == 432
    L0 = rt.layers[0]
    q, k, v = inputs[0][0]
    out = rt.layer_call(0, 0, q, k, v).clone()
    kw, vw = L0.k[:, :64 * P].clone(), L0.v[:, :64 * P].clone()
    for step in range(rt.cfg.steps + 1):
        for layer in range(rt.cfg.layers):
            if (step, layer) != (0, 0):
                rt.layer_call(step, layer, *inputs[step][layer])
    rt.commit_chunk(inputs)
    torch.cuda.synchronize()
    assert rt.dense_window() is False and rt.calls['dense'] > 0
    tiles = [0, 23, 48, 71]
    rows = torch.cat([torch.arange(t * 64, (t + 1) * 64) for t in tiles])
    want = ref.dense_attention(q[:, rows].cpu(), kw.cpu(), vw.cpu()).bfloat16().float()
    got = out[:, rows].cpu().float()
    err, mx = ref.rel_l2(got, want), float((got - want).abs().max())
    print(f"full-size dense call: rel-L2 {err:.3e} max-abs {mx:.3e}", flush=True)
    assert err <= 5e-3 and mx <= 2e-2
    order = rt.last_order.cpu()
    w = rt.group_weights
    pages = og.page_order(rt.cfg.history_pages)
    for layer in (1, 14, 29):
        want_o = og.group_order(inputs.clean_k[layer].cpu().transpose(0, 1), inputs.clean_v[layer].cpu().transpose(0, 1),
                                w.bank[layer].cpu(), w.group_v[layer].cpu(), w.gate[layer].cpu(), pages=pages)
        same = (order[layer].long() == want_o).all(-1)
        print(f"full-size commit, layer {layer}: {int(same.sum())}/12 heads in the oracle's order", flush=True)
        assert torch.equal(order[layer].long(), want_o)
