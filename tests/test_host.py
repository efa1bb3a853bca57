"""Host-side logic on the CPU: tier page counts, the Python wrappers' argument
checks, K/V stride detection, summary slab slicing, and the C ABI's own
argument checks (every rejected call returns hipErrorInvalidValue before any
HIP call, so these run without a GPU)."""
import ctypes
import os

import pytest
import torch

from streaming_sparse_amd import _lib, workload
from streaming_sparse_amd.attention import Workspace
from streaming_sparse_amd.legacy_components import attention, kv_strides
from streaming_sparse_amd.ops import Summary
from streaming_sparse_amd.route import route, select, tier_count

INVALID = 1   # hipErrorInvalidValue
H, D = 2, 128


def summary_slab(pages, cap=None):
    cap = cap or pages
    s = Summary(torch.zeros(H, cap, 4, D, dtype=torch.bfloat16), torch.zeros(H, cap, D, dtype=torch.bfloat16),
                torch.zeros(H, cap, 3, 8, dtype=torch.bfloat16), torch.zeros(H, cap, 4, 12, dtype=torch.bfloat16))
    return s.slice(0, pages)


def test_tier_counts():
    """Page counts of the reference tiers: floor(0.15 P) (VR/runtime.py:279-288),
    24 + n (VB/graph.py:210), max(1, floor(0.1 P)) (RV/ops.py:113-138)."""
    assert [tier_count('base', p) for p in (216, 288, 432, 504)] == [32, 43, 64, 75]
    assert tier_count('intersection', 432, 40) == 64
    assert [tier_count('topk', p) for p in (5, 216, 432)] == [1, 21, 43]
    with pytest.raises(ValueError):
        tier_count('dense', 432)


def test_summary_slice_keeps_slab_head_stride():
    s = summary_slab(100, cap=128)
    assert s.pages == 100 and s.head_pages == 128


def test_kv_strides_token_and_head_major():
    L = 64 * 3
    k = torch.zeros(1, L, H, D, dtype=torch.bfloat16)
    assert kv_strides(k, k.clone()) == (H * D, D)
    hm = torch.zeros(H, L, D, dtype=torch.bfloat16)
    kh = hm.transpose(0, 1)[None]
    assert kv_strides(kh, hm.clone().transpose(0, 1)[None]) == (D, L * D)
    with pytest.raises(ValueError):
        kv_strides(k[:, ::2], k[:, ::2])


def test_route_rejects_bad_arguments():
    s = summary_slab(216)
    q = torch.zeros(1, 128, H, D, dtype=torch.bfloat16)
    theta = torch.ones(H, 4)
    with pytest.raises(ValueError):
        route(q.float(), s, theta)                                   # q must be bf16
    with pytest.raises(ValueError):
        route(q[:, :, :, :64], s, theta)                              # head dim 128
    with pytest.raises(ValueError):
        route(q, s, theta, tier='intersection')                       # needs current_slots and n
    with pytest.raises(ValueError):
        route(q, summary_slab(72), theta, tier='base')                # base tier needs a history window
    with pytest.raises(ValueError):
        route(q, s, theta, rep_out=torch.zeros(H, 13, 512, dtype=torch.bfloat16))    # rep_out: ceil(216/16) tiles
    with pytest.raises(ValueError):
        route(q, s, theta, full_pset=[0])                             # Full_Pset only on the intersection tier
    with pytest.raises(ValueError):
        route(q, s, theta, lse_out=torch.zeros(H, 2, 8))              # lse_out shape
    with pytest.raises(ValueError):
        route(q, s, theta, tier='intersection', current_slots=[4, 4], n=216 - 23)   # n > P - 24
    with pytest.raises(ValueError):
        route(q, s, theta, tier='intersection', n=20)                 # current_slots needed unless P == 72


def test_attention_rejects_bad_arguments():
    p = 20
    s = summary_slab(p)
    q = torch.zeros(1, 128, H, D, dtype=torch.bfloat16)
    k = torch.zeros(1, 64 * p, H, D, dtype=torch.bfloat16)
    ids = torch.zeros(H, 2, 3, dtype=torch.int32)
    basis = torch.zeros(H, D, 8)
    ws = Workspace()
    with pytest.raises(ValueError):
        attention(q.transpose(1, 2).contiguous().transpose(1, 2), k, k, s, basis, ids, ws)   # q not contiguous
    with pytest.raises(ValueError):
        attention(q, k, k.float(), s, basis, ids, ws)                 # v must be bf16 like k
    with pytest.raises(ValueError):
        attention(q, k, k, s, basis, ids.long(), ws)                  # ids int32
    with pytest.raises(ValueError):
        attention(q, k, k, s, basis, ids[:, :1], ws)                  # ids [H, N/64, C]
    with pytest.raises((TypeError, ValueError)):
        bad = Summary(s.keys.float(), s.mean, s.detail, s.stats)
        attention(q, k, k, bad, basis, ids, ws)                       # summaries are bf16
    with pytest.raises(ValueError):
        attention(q, k, k, s, basis, ids, ws, all_pages=True)         # all_pages needs P entries per row


def test_risk_rejects_foreign_logits():
    """risk() consumes the reference's z only if it is the probe logits of
    its probes (checked on the host before any library call)."""
    from streaming_sparse_amd.legacy_components import risk
    p = 20
    g = torch.Generator().manual_seed(1)
    s = Summary(torch.randn(H, p, 4, D, generator=g).bfloat16(), torch.zeros(H, p, D, dtype=torch.bfloat16),
                torch.zeros(H, p, 3, 8, dtype=torch.bfloat16), torch.zeros(H, p, 4, 12, dtype=torch.bfloat16))
    probes = torch.randn(H, 2, 16, D, generator=g)
    z = torch.randn(H, 2, 16, p, 4, generator=g)
    with pytest.raises(ValueError):
        risk(probes, z, s, torch.ones(H, 4))                          # not the logits of these probes
    with pytest.raises(ValueError):
        risk(probes, z[..., :2], s, torch.ones(H, 4))                 # wrong shape


def test_quota_tables_keep_totals():
    """Seeded A/B tables: A + B constant over heads at every (step, layer)
    (VB/quota_counts.py:1-13)."""
    tab = workload.quota_table(2)
    tot = tab.sum(-1)
    assert bool((tot == tot[..., :1]).all()) and bool((tab[..., 0] >= 1).all())


@pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH), reason="libssattn.so not built")
def test_c_abi_rejects_bad_shapes():
    L = _lib.lib()
    N = None
    # ssa_attention: queries a multiple of 64, pages <= 512, count <= pages, K/V rows of 128 elements; the
    # general call needs page means, basis and ceil(pages/16) operand tiles, 16-byte aligned
    att = lambda n, pages, count, tok, mean=16, ops=16, tiles=27, flags=0: L.ssa_attention(
        N, N, N, N, mean, 16, ops, N, N, n, 12, pages, pages, tiles, count, tok, 128, flags, N, 0, N)
    assert att(65, 432, 64, 1536) == INVALID
    assert att(4608, 513, 64, 1536) == INVALID
    assert att(4608, 432, 433, 1536) == INVALID
    assert att(4608, 432, 64, 64) == INVALID
    assert att(4608, 432, 64, 1536, mean=None) == INVALID
    assert att(4608, 432, 64, 1536, ops=None) == INVALID
    assert att(4608, 432, 64, 1536, ops=24) == INVALID                # misaligned
    assert att(4608, 432, 64, 1536, tiles=26) == INVALID              # 432 pages need 27 tiles
    # a staged call (flags bit 2) is a general call and needs the workspace
    assert att(4608, 432, 432, 1536, flags=6) == INVALID
    assert att(4608, 432, 64, 1536, flags=5) == INVALID               # no workspace
    # the workspace size query rejects what the call rejects; a staged call keeps two states of
    # 33,280 bytes per tile
    wb = L.ssa_attention_workspace_bytes
    assert wb(65, 12, 432, 64, 1) == -1
    assert wb(4608, 12, 432, 433, 1) == -1
    assert wb(4608, 12, 432, 432, 6) == -1
    assert wb(4608, 12, 432, 64, 5) == 864 * 2 * 33280
    # ssa_route: pages in (0, 512], modes -1..2, base count >= 25, quota count = 24 + total,
    # operand tiles (when asked for) 16-byte aligned, ceil(pages/16) of them, with the detail rows
    rt = lambda pages, count, mode, total, cur=None, ops=None, det=None, tiles=32, eps=0.0, rows=None, cnt=None: \
        L.ssa_route(N, 128, 64 * 12 * 128, 12 * 128, 0, N, N, N, cur, N, N, N, N, N, 12, 72, pages, pages, count, mode,
                    total, det, ops, tiles, eps, rows, cnt, N)
    assert rt(0, 64, 0, 0) == INVALID
    assert rt(513, 64, 0, 0) == INVALID
    assert rt(432, 64, 3, 0) == INVALID
    assert rt(432, 24, 0, 0) == INVALID
    assert rt(72, 64, 0, 0) == INVALID
    assert rt(432, 60, 1, 40, cur=8) == INVALID
    assert rt(432, 64, 1, 40) == INVALID                              # no current quotas
    assert rt(216, 217, 2, 0) == INVALID                              # count > pages
    assert rt(216, 24 + 193, 1, 193, cur=8) == INVALID                # total > P - 24
    assert rt(432, 20, 1, -4, cur=8) == INVALID                       # negative total
    assert rt(80, 44, 1, 20, cur=8) == INVALID                        # 72 < P < 96: no such window
    assert rt(432, 64, 0, 0, ops=16, det=None) == INVALID             # operand tiles without detail rows
    assert rt(432, 64, 0, 0, ops=8, det=16) == INVALID                # misaligned
    assert rt(432, 64, 0, 0, ops=16, det=16, tiles=26) == INVALID     # 432 pages need 27 tiles
    assert rt(432, 64, 0, 0, rows=16) == INVALID                      # near-tie rows without their counter
    assert rt(432, 64, 0, 0, rows=16, cnt=16, eps=-1.0) == INVALID    # negative epsilon
    assert rt(432, 64, -1, 0, rows=16, cnt=16, eps=1e-3) == INVALID   # risk only: no selection
    # ssa_select: 0 < pages <= 512, 1 <= cap <= min(id_capacity, pages), density count <= id_capacity,
    # scores / own / outputs present (valid may be NULL)
    sel = lambda rows, pages, thr, fixed, cap, idcap, sc=8: L.ssa_select(sc, 8, N, rows, pages, 0.0, thr, fixed, cap,
                                                                           idcap, 8, 8, 8, 8, 8, N)
    assert sel(0, 410, 1, 41, 103, 128) == INVALID
    assert sel(6, 513, 1, 41, 103, 128) == INVALID
    assert sel(6, 410, 1, 41, 129, 128) == INVALID                    # cap > id_capacity
    assert sel(6, 90, 1, 9, 100, 128) == INVALID                      # cap > pages
    assert sel(6, 410, 1, 41, 0, 128) == INVALID
    assert sel(6, 410, 0, 0, 103, 128) == INVALID                     # density count < 1
    assert sel(6, 410, 0, 129, 103, 128) == INVALID                   # density count > id_capacity
    assert sel(6, 410, 1, 41, 103, 128, sc=None) == INVALID
    # ssa_summary: page range inside the slab, iters >= 1
    sm = lambda first, pages, iters, init: L.ssa_summary(N, N, 1536, 128, init, N, N, N, N, N, 432, 12, first, pages,
                                                         iters, N)
    assert sm(400, 72, 4, 16) == INVALID
    assert sm(360, 72, 0, 16) == INVALID
    assert sm(360, 72, 4, None) == INVALID
    # ssa_summary_write: both sources and both cache tensors given, same range checks
    sw = lambda sk, first: L.ssa_summary_write(sk, 16, 1536, 128, 16, 16, 1536, 128, 16, N, N, N, N, N, 432, 12,
                                               first, 72, 4, N)
    assert sw(None, 360) == INVALID
    assert sw(16, 400) == INVALID
    assert sw(8, 360) == INVALID                                       # source rows not 16-byte aligned
    # the layer-batched entries: 1..32 layers, non-null arrays and entries
    arr = lambda n, v=16: _lib.ptrs([None] * n) if v is None else (ctypes.c_void_p * n)(*([v] * n))
    sl = lambda n, a: L.ssa_summary_layers(n, a, a, 1536, 128, 16, a, a, a, a, a, 432, 12, 360, 72, 4, N)
    assert sl(0, arr(1)) == INVALID
    assert sl(33, arr(33)) == INVALID
    assert sl(2, arr(2, None)) == INVALID
    assert sl(2, None) == INVALID
    rb = lambda n, a: L.ssa_anchor_rebase_layers(n, a, 1536, 128, a, 1536, 128, 16, 32, 1536, 12, N)
    assert rb(33, arr(33)) == INVALID
    assert rb(2, arr(2, None)) == INVALID
    cm = lambda n, a: L.ssa_commit_pages_layers(n, a, a, 1536, 128, a, 72, 16, 432, a, a, 1536, 128, 12, N)
    assert cm(0, arr(1)) == INVALID
    assert cm(2, arr(2, None)) == INVALID
    el = lambda n, a: L.ssa_encode_layers(n, a, a, a, a, 432, a, N, N, N, N, N, N, N, a, a, a, 432, 12, 360, 72, 256,
                                          N)
    assert el(33, arr(33)) == INVALID
    assert el(2, arr(2, None)) == INVALID
    # ssa_encode: hidden width <= 256, page range inside both slabs
    en = lambda pages, hidden: L.ssa_encode(N, N, N, N, 432, N, N, N, N, N, N, N, N, N, N, N, 432, 12, 360, pages,
                                            hidden, N)
    assert en(73, 256) == INVALID
    assert en(72, 257) == INVALID
    # ssa_pset: a 72-page window (the first chunk, 24 <= count <= 72) or 96 < pages <= 512 with
    # 1 <= count <= pages.  Every pointer the check requires is given (never dereferenced: the call
    # returns before any launch), so the shapes alone decide.
    D = ctypes.c_void_p(256)
    ps = lambda pages, count, heads=D: L.ssa_pset(N, 128, 64 * 12 * 128, 12 * 128, 0, N, pages, N, N, N, pages, N,
                                                  N, D, N, N, N, heads, 3, D, D, D, D, D, N, D, 12, 72, pages,
                                                  count, N)
    assert ps(96, 40) == INVALID                                      # no history partition
    assert ps(80, 40) == INVALID
    assert ps(513, 40) == INVALID
    assert ps(72, 73) == INVALID
    assert ps(72, 23) == INVALID                                      # fewer than the 24 anchors
    assert ps(432, 433) == INVALID
    assert ps(432, 0) == INVALID
    assert ps(432, 64, heads=N) == INVALID
    # ssa_rep_operands: heads >= 1, pages in (0, 512], ceil(pages/16) tiles, aligned output
    ro = lambda heads, pages, tiles, out=16: L.ssa_rep_operands(16, out, heads, pages, 512, tiles, N)
    assert ro(0, 432, 27) == INVALID
    assert ro(12, 513, 33) == INVALID
    assert ro(12, 432, 26) == INVALID
    assert ro(12, 432, 27, out=8) == INVALID
    assert ro(12, 432, 27, out=None) == INVALID


def test_select_rejects_bad_config():
    """select checks the reference Config's invariants
    (RV/ops.py:21-24) before it calls the library."""
    from types import SimpleNamespace
    scores = torch.zeros(1, 1, 410)
    own = torch.zeros(1, 1, dtype=torch.int32)
    with pytest.raises(ValueError):
        select(scores, own, SimpleNamespace(density=0.3, max_fraction=0.25, id_capacity=128))
    with pytest.raises(ValueError):
        select(scores, own, SimpleNamespace(density=0.1, max_fraction=0.25, id_capacity=100))
    with pytest.raises(ValueError):
        select(torch.zeros(1, 1, 600), own, id_capacity=200)



def test_batch_graphs_checks_call_shape():
    """BatchGraphs rejects an unknown tier, a q outside the reference's
    [H, T, 64 or 16, 128] block layout, and an intersection call without its
    quota, before any device work."""
    from streaming_sparse_amd.graph import BatchGraphs
    with pytest.raises(ValueError):
        BatchGraphs('nope')
    p = 216
    s = Summary(torch.zeros(H, p, 4, D, dtype=torch.bfloat16), torch.zeros(H, p, D, dtype=torch.bfloat16),
                torch.zeros(H, p, 3, 8, dtype=torch.bfloat16), torch.zeros(H, p, 4, 12, dtype=torch.bfloat16))
    bg = BatchGraphs('intersection')
    with pytest.raises(ValueError):
        bg.get(torch.zeros(H, 72, 32, D), s, None, torch.ones(H, 4), None, None, False)
    with pytest.raises(ValueError):                                  # n and current_slots not set
        bg.get(torch.zeros(H, 72, 64, D), s, None, torch.ones(H, 4), None, None, False)
    bg.n = 40
    bg.current_slots = torch.full((H,), 10)
    with pytest.raises(ValueError):                                  # Full_Pset without reader / encoding
        bg.get(torch.zeros(H, 72, 64, D), s, None, torch.ones(H, 4), None, None, True, [3])
