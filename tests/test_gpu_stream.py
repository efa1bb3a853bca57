"""The rolling-window runtime on the GPU: a 3-layer stack with a 168-page
history ring (window up to 240 pages), one denoise step plus the clean step
per chunk, Full_Pset on layer 2, run for 8 chunks so that the ring wraps
(from the third commit) and the anchor is rebased (chunks 6 and 7).

Checks against the oracle on the runtime's own state:
* every history page of the ring holds, bit for bit, the K/V rows of the
  grouped chunk page that the ring's slot sequence put there last (each
  head's rows in that head's grouped token order, a permutation of the
  chunk; the first chunk's anchor frame fills pages 0..23);
* the anchor frame's keys are the chunk-0 keys rebased by 3c - 15 frames
  (oracle shift_temporal, bit for bit), its values untouched, and its page
  summaries are the summary oracle's of the rebased keys;
* after the wrap and the rebase, a dense call (layer 0), a sparse call
  (layer 1) and a Full_Pset-corrected sparse call (layer 2) against softmax
  attention and SelectedAttention.fixed on the page tables they used."""
import pytest
import torch

from oracle import reference as ref
from oracle import summary as osum
from streaming_sparse_amd import workload
from streaming_sparse_amd.ops import Summary
from streaming_sparse_amd.runtime import ANCHOR_TOKENS, CURRENT, StreamConfig, StreamRuntime, rebase_offset

pytestmark = pytest.mark.gpu
REL_L2, MAX_ABS = 5e-3, 2e-2
TILES = [0, 17, 40, 71]


def _check(got, want, tag):
    g, w = got.detach().cpu().float(), want.float()
    err = ref.rel_l2(g, w)
    mx = float((g - w).abs().max())
    print(f"{tag}: rel-L2 {err:.3e} max-abs {mx:.3e}", flush=True)
    assert err <= REL_L2 and mx <= MAX_ABS, (tag, err, mx)


def test_rolling_window(device):
    cfg = StreamConfig(layers=3, steps=1, history_pages=168, pset_layers=(2,), seed=8)
    rt = StreamRuntime(cfg, device)
    committed = {}          # chunk -> layer-1 clean-step (k, v) in its grouped order, on the CPU
    owner = {}              # ring page -> (chunk, chunk page)
    heads = torch.arange(12)
    for c in range(7):
        inputs = rt.chunk_inputs()
        slots = rt.ring.commit_slots()
        rt.run_chunk(inputs)
        torch.cuda.synchronize()
        k1, v1 = inputs[cfg.steps][1][1:]
        order = rt.last_order[1].cpu().long()                      # [H, 4608]
        assert torch.equal(order.sort(-1).values, torch.arange(4608).expand(12, -1))
        grouped = lambda x: x.cpu()[order.t(), heads[None, :]]    # row j, head h <- token order[h, j]
        committed[c] = (grouped(k1), grouped(v1))
        if c == 0:
            assert bool((order[:, :ANCHOR_TOKENS] < ANCHOR_TOKENS).all())   # anchor frame in pages 0..23
            anchor_k0, anchor_v = (x[:ANCHOR_TOKENS].clone() for x in committed[0])
        for j, s in enumerate(slots):
            owner[s] = (c, j)
        print(f"chunk {c}: history {rt.ring.n} pages, calls {rt.calls}", flush=True)
    assert rt.ring.n == 168 and rt.ring.commits == 7
    L1 = rt.layers[1]
    kc, vc = L1.k[0].cpu(), L1.v[0].cpu()
    # ring contents: pages 24..167 hold the last writer's grouped rows
    for s in range(24, 168):
        c, j = owner[s]
        k, v = committed[c]
        assert torch.equal(kc[64 * s:64 * s + 64].view(torch.int16), k[64 * j:64 * j + 64].view(torch.int16)), s
        assert torch.equal(vc[64 * s:64 * s + 64].view(torch.int16), v[64 * j:64 * j + 64].view(torch.int16)), s
    assert {owner[s][0] for s in range(24, 168)} == {5, 6}     # the 144-page span holds the last two chunks
    # anchor: chunk-0 keys rebased for chunk 6 (3 frames), values untouched
    freqs = workload.rope_table(128)
    want_k = ref.shift_temporal(anchor_k0[None], ANCHOR_TOKENS, freqs, rebase_offset(6))[0]
    assert torch.equal(kc[:ANCHOR_TOKENS].view(torch.int16), want_k.view(torch.int16))
    assert torch.equal(vc[:ANCHOR_TOKENS].view(torch.int16), anchor_v.view(torch.int16))
    assert not torch.equal(kc[:ANCHOR_TOKENS], anchor_k0)

    # chunk 7: rebase by 6 frames, then one call of each kind after the wrap
    inputs = rt.chunk_inputs()
    rt.begin_chunk()
    torch.cuda.synchronize()
    want_k = ref.shift_temporal(anchor_k0[None], ANCHOR_TOKENS, freqs, rebase_offset(7))[0]
    assert torch.equal(L1.k[0, :ANCHOR_TOKENS].cpu().view(torch.int16), want_k.view(torch.int16))
    # anchor summaries rebuilt from the rebased keys
    kp = want_k.transpose(0, 1).reshape(12, 24, 64, 128)
    vp = anchor_v.transpose(0, 1).reshape(12, 24, 64, 128)
    wsum = osum.summaries(kp, vp, L1.basis.cpu().float(), rt.init[:, :24].cpu())
    ok = wsum['margin'] > 1e-5
    for name in ('keys', 'mean'):
        got = getattr(L1.slab, name)[:, :24].cpu().float()[ok]
        w = wsum[name].float()[ok]
        assert bool(((got - w).abs() <= w.abs() * 2.0 ** -7 + 1e-6).all()), name
    P = rt.ring.n + CURRENT
    rows = torch.cat([torch.arange(t * 64, (t + 1) * 64) for t in TILES])
    for layer in range(3):
        q, k, v = inputs[0][layer]
        out = rt.layer_call(0, layer, q, k, v).clone()
        torch.cuda.synchronize()
        L = rt.layers[layer]
        kw, vw = L.k[:, :64 * P].cpu(), L.v[:, :64 * P].cpu()
        if layer == 0:
            hs = [0, 7]
            want = ref.dense_attention(q[:, rows][:, :, hs].cpu(), kw[:, :, hs], vw[:, :, hs]).bfloat16()
            _check(out[:, rows][:, :, hs], want, "post-wrap dense layer")
            continue
        ids = rt.last_ids.cpu()
        assert (ids[..., 0] == torch.arange(72) + P - 72).all()
        s = Summary(*(getattr(L.slab, f)[:, :P].cpu() for f in Summary.FIELDS))
        want = ref.selected_attention(q.cpu(), kw, vw, s, L.basis.cpu().float(), ids, tiles=TILES).bfloat16()
        _check(out[:, rows], want[:, rows], f"post-wrap sparse layer {layer}")
        # the call's current-page summaries are the summary oracle's of the chunk's K/V
        kp = k.cpu().transpose(0, 1).reshape(12, 72, 64, 128)
        vp = v.cpu().transpose(0, 1).reshape(12, 72, 64, 128)
        wsum = osum.summaries(kp, vp, L.basis.cpu().float(), rt.init.cpu())
        ok = wsum['margin'] > 1e-5
        for name in ('keys', 'mean'):
            got = getattr(s, name)[:, P - 72:].float()[ok]
            w = wsum[name].float()[ok]
            assert bool(((got - w).abs() <= w.abs() * 2.0 ** -7 + 1e-6).all()), (layer, name)
    assert rt.calls['full_pset'] >= 1


def test_first_chunk_sparse(device):
    """sparse_start_chunks=(0,): chunk 0 runs sparse on its 72-page window
    (the reference's first-chunk quota n = 4, A = 4: VB/queue_policy.py:
    25-28) with Full_Pset on layer 2, chunk 1 dense; the chunk-0 sparse and
    corrected calls match SelectedAttention.fixed on their page tables."""
    cfg = StreamConfig(layers=3, steps=1, history_pages=168, pset_layers=(2,), seed=9, sparse_start_chunks=(0,))
    rt = StreamRuntime(cfg, device)
    inputs = rt.chunk_inputs()
    rt.begin_chunk()
    rows = torch.cat([torch.arange(t * 64, (t + 1) * 64) for t in TILES])
    for layer in range(3):
        q, k, v = inputs[0][layer]
        out = rt.layer_call(0, layer, q, k, v).clone()
        torch.cuda.synchronize()
        if layer == 0:
            continue
        L = rt.layers[layer]
        ids = rt.last_ids.cpu()
        assert ids.shape[-1] == 28 and (ids[..., 0] == torch.arange(72)).all()
        kw, vw = L.k[:, :64 * 72].cpu(), L.v[:, :64 * 72].cpu()
        s = Summary(*(getattr(L.slab, f)[:, :72].cpu() for f in Summary.FIELDS))
        want = ref.selected_attention(q.cpu(), kw, vw, s, L.basis.cpu().float(), ids, tiles=TILES).bfloat16()
        _check(out[:, rows], want[:, rows], f"first-chunk sparse layer {layer}")
    assert rt.calls == dict(sparse=2, dense=1, full_pset=1)
    # the rest of chunk 0 (clean step, commit) and chunk 1 (dense: 72 history pages)
    for layer in range(3):
        rt.layer_call(cfg.steps, layer, *inputs[cfg.steps][layer])
    rt.commit_chunk(inputs)
    rt.end_chunk()
    rt.run_chunk(rt.chunk_inputs())
    torch.cuda.synchronize()
    assert rt.ring.n == 144 and rt.calls['sparse'] == 2 and rt.calls['full_pset'] == 1
    assert bool(torch.isfinite(rt.last['out'].float()).all())


def test_base_tier_stream(device):
    """The base tier as a stream (the 116-call base workload of a chunk,
    here 3 layers x 1 step): chunks 0-1 dense, chunk 2 sparse on a 216-page
    window with the base table (own, 24 anchors, the 7 highest-risk other
    pages: floor(0.15 P) = 32); the page tables equal the oracle's base
    selection off near ties, and the calls match SelectedAttention.fixed on
    their tables."""
    cfg = StreamConfig(layers=3, steps=1, history_pages=168, pset_layers=(2,), seed=10, tier='base')
    rt = StreamRuntime(cfg, device)
    for c in range(2):
        rt.run_chunk(rt.chunk_inputs())
    assert rt.calls['sparse'] == 0
    inputs = rt.chunk_inputs()
    rt.begin_chunk()
    P = rt.ring.n + CURRENT
    assert P == 216
    rows = torch.cat([torch.arange(t * 64, (t + 1) * 64) for t in TILES])
    for layer in (1, 2):
        q, k, v = inputs[0][layer]
        out = rt.layer_call(0, layer, q, k, v).clone()
        torch.cuda.synchronize()
        L = rt.layers[layer]
        ids = rt.last_ids.cpu()
        assert ids.shape[-1] == 32
        s = Summary(*(getattr(L.slab, f)[:, :P].cpu() for f in Summary.FIELDS))
        own = (torch.arange(72) + P - 72)[None].expand(12, -1)
        pr = ref.probes(q.cpu())
        r64 = ref.risk(pr, ref.route_logits(pr, s.keys, torch.float64), s.stats, rt.theta.cpu(), dtype=torch.float64)
        want = ref.select_base(r64, own, 32)
        cand = r64.clone()
        cand[..., :24] = -float("inf")
        cand.scatter_(-1, own[..., None], -float("inf"))
        ties = ref.near_tie_rows(cand, torch.full(own.shape, 7))
        same_set = (ids.sort(-1).values == want.sort(-1).values).all(-1)
        print(f"base stream layer {layer}: {int(same_set.sum())}/864 tables equal, {int(ties.sum())} near-tie rows",
              flush=True)
        assert bool((same_set | ties).all())
        kw, vw = L.k[:, :64 * P].cpu(), L.v[:, :64 * P].cpu()
        want_out = ref.selected_attention(q.cpu(), kw, vw, s, L.basis.cpu().float(), ids, tiles=TILES).bfloat16()
        _check(out[:, rows], want_out[:, rows], f"base stream layer {layer}")
    assert rt.calls['sparse'] == 2 and rt.calls['full_pset'] == 0
