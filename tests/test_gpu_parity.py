"""HIP path vs. the CPU oracle on identical seeded inputs.

Bar (north-star): page tables bit-exact except rows whose selection boundary
is a near tie (two risk scores within 1e-3 relative); attention outputs within
rel-L2 5e-3 and max-abs 2e-2 of the oracle's bf16-rounded output."""
import functools
import math

import pytest
import torch

from oracle import reference as ref
from streaming_sparse_amd import workload
from streaming_sparse_amd.attention import Workspace
from streaming_sparse_amd.legacy_components import attention, risk as risk_fn
from streaming_sparse_amd.ops import Summary
from streaming_sparse_amd.route import route

pytestmark = pytest.mark.gpu
REL_L2, MAX_ABS = 5e-3, 2e-2


@functools.lru_cache(maxsize=None)
def call_inputs(cfg, frames, heads=12):
    return workload.make_call(cfg, frames, heads=heads)


def oracle_risk(x):
    pr = ref.probes(x.q)
    return ref.risk(pr, ref.route_logits(pr, x.summary.keys), x.summary.stats, x.theta)


def check_out(got, want, tag=""):
    g = got.detach().cpu().float()
    w = want.float()
    err = ref.rel_l2(g, w)
    mx = float((g - w).abs().max())
    print(f"{tag} rel-L2 {err:.3e} max-abs {mx:.3e}", flush=True)
    assert torch.isfinite(g).all()
    assert err <= REL_L2 and mx <= MAX_ABS, (tag, err, mx)
    return err, mx


def test_risk_matches_oracle(device):
    x = call_inputs(0, 9)
    g = x.to(device)
    pr = ref.probes(x.q)
    got = risk_fn(ref.probes(g.q), None, g.summary, g.theta).cpu()
    want = ref.risk(pr, ref.route_logits(pr, x.summary.keys, torch.float64), x.summary.stats, x.theta,
                    dtype=torch.float64)
    rel = ((got.double() - want).abs() / want.abs().clamp_min(1e-30)).max()
    print("risk max rel err", float(rel), flush=True)
    assert rel < 1e-4


@pytest.mark.parametrize("pages", [8, 20, 72])
def test_risk_small_windows(device, pages):
    """Windows of fewer than 32 pages leave some of the router's waves with
    no tile of their own, and 20 pages end in a partial tile; 72 is the first
    chunk's window (VB/graph.py:143-148)."""
    x = call_inputs(0, 9)
    sub = x.summary.slice(0, pages)
    pr = ref.probes(x.q)
    got = risk_fn(ref.probes(x.q.to(device)), None, Summary(*(t.to(device) for t in
                                                               (x.summary.keys, x.summary.mean, x.summary.detail,
                                                                x.summary.stats))).slice(0, pages),
                  x.theta.to(device)).cpu()
    want = ref.risk(pr, ref.route_logits(pr, sub.keys, torch.float64), sub.stats, x.theta, dtype=torch.float64)
    assert got.shape == (12, 72, pages)
    rel = ((got.double() - want).abs() / want.abs().clamp_min(1e-30)).max()
    print(f"P={pages} risk max rel err {float(rel):.3e}", flush=True)
    assert rel < 1e-4


@pytest.mark.parametrize("cfg,frames", [(0, 9), (1, 18)])
def test_route_base_matches_oracle(device, cfg, frames):
    x = call_inputs(cfg, frames)
    g = x.to(device)
    ids, mask, risk, _ = route(g.q, g.summary, g.theta, tier='base', own=g.own)
    P = x.pages
    count = P * 15 // 100
    r64 = ref.risk(ref.probes(x.q), ref.route_logits(ref.probes(x.q), x.summary.keys, torch.float64),
                   x.summary.stats, x.theta, dtype=torch.float64)
    rel = float(((risk.cpu().double() - r64).abs() / r64.abs().clamp_min(1e-30)).max())
    assert rel < 1e-4, rel
    want = ref.select_base(r64, x.own, count)
    cand = r64.clone()
    cand[..., :24] = -math.inf
    cand.scatter_(-1, x.own[..., None], -math.inf)
    ties = ref.near_tie_rows(cand, torch.full(x.own.shape, count - 25))
    got = ids.cpu()
    same = (got == want).all(-1)
    # rows whose ranked part holds near-equal risks may order those pages
    # differently, with the same page set, in the kernel's own risk order
    order_ties = ref.near_tie_order_rows(r64, want, 25)
    same_set = (got.sort(-1).values == want.sort(-1).values).all(-1)
    print(f"P={P}: {int(same.sum())}/{same.numel()} rows identical, {int(ties.sum())} near-tie rows, "
          f"{int((order_ties & ~same).sum())} rows reordered among near-equal risks", flush=True)
    assert bool((same | ties | (order_ties & same_set)).all())
    ranked = risk.cpu().gather(-1, got[..., 25:].long())
    assert bool((ranked[..., :-1] >= ranked[..., 1:]).all())
    # near-tie rows still keep the invariants
    assert (got[..., 0] == x.own).all() and (got[..., 1:25] == torch.arange(24)).all()
    assert (got.sort(-1).values.diff(dim=-1) > 0).all()
    assert torch.equal(mask.cpu(), ref.mask_from_ids(got, P))


def test_route_topk_matches_oracle(device):
    """Fixed top-floor(0.1 P) with own forced (mode 2)."""
    x = call_inputs(0, 9)
    g = x.to(device)
    ids, mask, risk, _ = route(g.q, g.summary, g.theta, tier='topk', own=g.own)
    P = x.pages
    r64 = ref.risk(ref.probes(x.q), ref.route_logits(ref.probes(x.q), x.summary.keys, torch.float64),
                   x.summary.stats, x.theta, dtype=torch.float64)
    count = max(1, int(P * 0.1))
    want, want_mask = ref.select_topk(r64, x.own, count)
    cand = r64.scatter(-1, x.own[..., None], -math.inf)
    ties = ref.near_tie_rows(cand, torch.full(x.own.shape, count - 1))
    got = ids.cpu()
    same = (got == want).all(-1)
    order_ties = ref.near_tie_order_rows(r64, want, 1)
    same_set = (got.sort(-1).values == want.sort(-1).values).all(-1)
    print(f"topk: {int(same.sum())}/{same.numel()} rows identical, {int(ties.sum())} near-tie rows", flush=True)
    assert bool((same | ties | (order_ties & same_set)).all())
    assert (got[..., 0] == x.own).all()
    assert torch.equal(mask.cpu(), ref.mask_from_ids(got, P))
    assert bool((mask.cpu() == want_mask)[~ties].all())


@pytest.mark.parametrize("blocks", [3, 5])
def test_route_odd_blocks(device, blocks):
    """An odd number of query blocks leaves the router's last workgroup one
    block; base tier on the first `blocks` blocks of the 216-page call."""
    x = call_inputs(0, 9)
    q = x.q[:, :64 * blocks].contiguous()
    own = x.own[:, :blocks].contiguous()
    g = x.to(device)
    ids, mask, risk, _ = route(q.to(device), g.summary, g.theta, tier='base', own=own.to(device))
    P = x.pages
    count = P * 15 // 100
    r64 = ref.risk(ref.probes(q), ref.route_logits(ref.probes(q), x.summary.keys, torch.float64),
                   x.summary.stats, x.theta, dtype=torch.float64)
    assert risk.shape == (12, blocks, P)
    rel = float(((risk.cpu().double() - r64).abs() / r64.abs().clamp_min(1e-30)).max())
    assert rel < 1e-4, rel
    want = ref.select_base(r64, own, count)
    cand = r64.clone()
    cand[..., :24] = -math.inf
    cand.scatter_(-1, own[..., None], -math.inf)
    ties = ref.near_tie_rows(cand, torch.full(own.shape, count - 25))
    got = ids.cpu()
    same = (got == want).all(-1)
    order_ties = ref.near_tie_order_rows(r64, want, 25)
    same_set = (got.sort(-1).values == want.sort(-1).values).all(-1)
    print(f"blocks={blocks}: {int(same.sum())}/{same.numel()} rows identical, {int(ties.sum())} near-tie rows",
          flush=True)
    assert bool((same | ties | (order_ties & same_set)).all())
    assert torch.equal(mask.cpu(), ref.mask_from_ids(got, P))


def test_route_intersection_matches_oracle(device):
    x = call_inputs(2, 18)
    g = x.to(device)
    tab = workload.quota_table(2)
    a = tab[0, 3, :, 0]
    n = int(tab[0, 3, 0].sum())
    ids, mask, risk, _ = route(g.q, g.summary, g.theta, tier='intersection', own=g.own, current_slots=a, n=n)
    P = x.pages
    r64 = ref.risk(ref.probes(x.q), ref.route_logits(ref.probes(x.q), x.summary.keys, torch.float64),
                   x.summary.stats, x.theta, dtype=torch.float64)
    want_mask = ref.quota_mask(r64, x.own, a, n)
    want = ref.lut(r64, want_mask, x.own, 24 + n)
    got_mask = mask.cpu()
    # near ties at either partition boundary
    hist = r64.clone()
    hist[..., :24] = -math.inf
    hist[..., P - 72:] = -math.inf
    cur = r64.clone()
    cur[..., :P - 72] = -math.inf
    cur.scatter_(-1, x.own[..., None], math.inf)
    ties = ref.near_tie_rows(hist, (n - a)[:, None].expand_as(x.own)) | \
        ref.near_tie_rows(cur, a[:, None].expand_as(x.own))
    same = (got_mask == want_mask).all(-1)
    print(f"intersection: {int(same.sum())}/{same.numel()} masks identical, {int(ties.sum())} near-tie rows",
          flush=True)
    assert bool((same | ties).all())
    got = ids.cpu()
    assert (got[..., 0] == x.own).all()
    assert torch.equal(ref.mask_from_ids(got, P), got_mask)
    # order: own first then descending risk (ties may swap neighbours)
    rows = same & ~ties
    rk = r64.gather(-1, got[..., 1:].long())
    assert (rk[..., :-1] >= rk[..., 1:] - 1e-6 * rk.abs()[..., 1:]).all()
    assert torch.equal(got[rows].sort(-1).values, want[rows].sort(-1).values)
    assert (mask.cpu()[..., :24]).all() and (got_mask[..., P - 72:].sum(-1) == a[:, None]).all()


def operand_tiles(detail, pages):
    """The detail operand tiles [H, ceil(P/16), 512] that ssa_rep_operands
    documents, restated with index arithmetic on the CPU: element j of chunk
    ((pair*2 + hh)*8 + rank)*2 + m of tile rt is detail[page, a, rank] with
    v = (8m + j) mod 12, page = 16 rt + 8 pair + 2 (v // 3) + hh, a = v % 3,
    and 0 for pages >= P."""
    h = detail.shape[0]
    tiles = (pages + 15) // 16
    out = torch.zeros(h, tiles, 2, 2, 8, 2, 8, dtype=torch.bfloat16)
    for rt in range(tiles):
        for pair in range(2):
            for hh in range(2):
                for m in range(2):
                    for j in range(8):
                        v = (8 * m + j) % 12
                        pg = 16 * rt + 8 * pair + 2 * (v // 3) + hh
                        if pg < pages:
                            out[:, rt, pair, hh, :, m, j] = detail[:, pg, v % 3, :]
    return out.reshape(h, tiles, 512)


@pytest.mark.parametrize("cfg,frames", [(0, 9), (1, 18)])
def test_route_writes_rep_operands(device, cfg, frames):
    """The router's side output of detail operand tiles equals the standalone
    kernel bit for bit (into a slab wider than the window), both equal the
    documented layout restated on the CPU, and the attention call that reads
    them equals the one that computes its own."""
    from streaming_sparse_amd.legacy_components import rep_operands
    x = call_inputs(cfg, frames)
    g = x.to(device)
    P = x.pages
    T = (P + 15) // 16
    basis = g.basis.to(torch.bfloat16).contiguous()
    want = rep_operands(g.summary, P, torch.empty(12, T, 512, device=device, dtype=torch.bfloat16))
    slab = torch.full((12, T + 2, 512), float("nan"), device=device, dtype=torch.bfloat16)
    ids, _, _, _ = route(g.q, g.summary, g.theta, tier='base', own=g.own, rep_out=slab)
    assert torch.equal(slab[:, :T].view(torch.int16), want.view(torch.int16))
    assert bool(slab[:, T:].isnan().all())           # tiles past the window untouched
    layout = operand_tiles(x.summary.detail[:, :P], P)
    assert torch.equal(want.cpu().view(torch.int16), layout.view(torch.int16))
    ws = Workspace()
    a = attention(g.q, g.k, g.v, g.summary, basis, ids, ws).clone()
    b = attention(g.q, g.k, g.v, g.summary, basis, ids, ws, rep_ops=slab)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("single", [False, True])
def test_attention_config0(device, single):
    """216-page window, base tier LUT (32 pages), all 72 query blocks x 12
    heads; the reference's two-term P.V (default) and the single-term opt-in."""
    x = call_inputs(0, 9)
    g = x.to(device)
    ids = ref.select_base(oracle_risk(x), x.own, 32)
    out = attention(g.q, g.k, g.v, g.summary, g.basis, ids.to(device), Workspace(), single_av=single)
    torch.cuda.synchronize()
    want = ref.selected_attention(x.q, x.k, x.v, x.summary, x.basis, ids).bfloat16()
    check_out(out, want, f"config0 single={single}")


TILES8 = [0, 9, 23, 35, 36, 50, 64, 71]


def tile_rows(tiles):
    return torch.cat([torch.arange(t * 64, (t + 1) * 64) for t in tiles])


@pytest.mark.parametrize("single", [False, True])
def test_attention_config1_tiles(device, single):
    """432-page window, 64 exact pages; oracle on 8 spread query blocks."""
    x = call_inputs(1, 18)
    g = x.to(device)
    ids = ref.select_base(oracle_risk(x), x.own, 64)
    out = attention(g.q, g.k, g.v, g.summary, g.basis, ids.to(device), Workspace(), single_av=single)
    torch.cuda.synchronize()
    want = ref.selected_attention(x.q, x.k, x.v, x.summary, x.basis, ids, tiles=TILES8).bfloat16()
    rows = tile_rows(TILES8)
    check_out(out[:, rows], want[:, rows], f"config1 tiles single={single}")


@pytest.mark.parametrize("single", [False, True])
def test_attention_config2_intersection_tiles(device, single):
    """432-page window under the intersection tier's per-head quotas (layer 3,
    step 0 of the seeded table: 24 anchors + A current + B history pages per
    head, A+B equal over the heads): the oracle's quota mask and LUT, then
    attention against the oracle on 8 spread query blocks; and the GPU
    router's own table through the same attention."""
    x = call_inputs(2, 18)
    g = x.to(device)
    tab = workload.quota_table(2)
    a = tab[0, 3, :, 0]
    n = int(tab[0, 3, 0].sum())
    r = oracle_risk(x)
    ids = ref.lut(r, ref.quota_mask(r, x.own, a, n), x.own, 24 + n)
    assert bool((ids >= 0).all())
    out = attention(g.q, g.k, g.v, g.summary, g.basis, ids.to(device), Workspace(), single_av=single)
    torch.cuda.synchronize()
    want = ref.selected_attention(x.q, x.k, x.v, x.summary, x.basis, ids, tiles=TILES8).bfloat16()
    rows = tile_rows(TILES8)
    check_out(out[:, rows], want[:, rows], f"config2 oracle table single={single}")
    ws = Workspace()
    gids, _, _, _ = route(g.q, g.summary, g.theta, tier='intersection', own=g.own, current_slots=a, n=n,
                          workspace=ws)
    out2 = attention(g.q, g.k, g.v, g.summary, g.basis, gids, ws, single_av=single)
    torch.cuda.synchronize()
    want2 = ref.selected_attention(x.q, x.k, x.v, x.summary, x.basis, gids.cpu(), tiles=TILES8).bfloat16()
    check_out(out2[:, rows], want2[:, rows], f"config2 router table single={single}")


@pytest.mark.parametrize("single", [False, True])
def test_full_call_properties(device, single):
    """Size-independent properties of the whole base call at its full size
    (432 pages, 12 heads, 4608 queries), where the oracle would take minutes:
    - two calls on the same inputs give bit-identical risk, page tables,
      detail operand tiles and outputs (no atomics or order-dependent
      reductions);
    - scaling V, the page V means and the V details by 2 scales every operand
      tile and every output by exactly 2 (the compensated and exact parts are
      linear in V, and a power of two commutes with every rounding);
    - reversing the order of each row's pages after its own page changes the
      output only by the online softmax's rounding, well inside the parity bar."""
    x = call_inputs(1, 18)
    g = x.to(device)
    basis = g.basis.to(torch.bfloat16).contiguous()
    ws = Workspace()

    def call(v, s):
        vrep = torch.empty(12, (x.pages + 15) // 16, 512, device=device, dtype=torch.bfloat16)
        ids, _, risk, _ = route(g.q, s, g.theta, tier='base', own=g.own, workspace=ws, rep_out=vrep)
        out = attention(g.q, g.k, v, s, basis, ids, ws, rep_ops=vrep, single_av=single).clone()
        return ids.clone(), risk.clone(), vrep, out

    ids, risk, vrep, out = call(g.v, g.summary)
    ids2, risk2, vrep2, out2 = call(g.v, g.summary)
    torch.cuda.synchronize()
    assert torch.equal(ids, ids2) and torch.equal(risk, risk2)
    assert torch.equal(vrep, vrep2) and torch.equal(out, out2)
    assert ids.shape == (12, 72, 64) and bool(torch.isfinite(out.float()).all())

    s2 = Summary(g.summary.keys, g.summary.mean * 2, g.summary.detail * 2, g.summary.stats)
    ids3, risk3, vrep3, out3 = call(g.v * 2, s2)
    torch.cuda.synchronize()
    assert torch.equal(ids3, ids) and torch.equal(risk3, risk)
    assert torch.equal(vrep3, vrep * 2) and torch.equal(out3, out * 2)

    rev = torch.cat([ids[..., :1], ids[..., 1:].flip(-1)], -1).contiguous()
    out4 = attention(g.q, g.k, g.v, g.summary, basis, rev, ws, rep_ops=vrep, single_av=single).clone()
    torch.cuda.synchronize()
    check_out(out4, out.cpu(), "reversed page order")


def test_route_and_attention_largest_window(device):
    """504 pages (21 frames), the largest window of whole frames under the
    512-page limit: the router's waves hold 15 or 16 tiles, the attention
    walks 75 exact pages (C = 15% of P) and up to 32 rep tiles, the last one half
    beyond the window."""
    x = call_inputs(1, 21)
    g = x.to(device)
    P = x.pages
    assert P == 504
    count = P * 15 // 100
    ws = Workspace()
    basis = g.basis.to(torch.bfloat16).contiguous()
    vrep = torch.empty(12, (P + 15) // 16, 512, device=device, dtype=torch.bfloat16)
    ids, mask, risk, _ = route(g.q, g.summary, g.theta, tier='base', own=g.own, workspace=ws, rep_out=vrep)
    out = attention(g.q, g.k, g.v, g.summary, basis, ids, ws, rep_ops=vrep)
    torch.cuda.synchronize()
    r64 = ref.risk(ref.probes(x.q), ref.route_logits(ref.probes(x.q), x.summary.keys, torch.float64),
                   x.summary.stats, x.theta, dtype=torch.float64)
    rel = float(((risk.cpu().double() - r64).abs() / r64.abs().clamp_min(1e-30)).max())
    assert rel < 1e-4, rel
    want_ids = ref.select_base(r64, x.own, count)
    cand = r64.clone()
    cand[..., :24] = -math.inf
    cand.scatter_(-1, x.own[..., None], -math.inf)
    ties = ref.near_tie_rows(cand, torch.full(x.own.shape, count - 25))
    got = ids.cpu()
    same = (got == want_ids).all(-1)
    order_ties = ref.near_tie_order_rows(r64, want_ids, 25)
    same_set = (got.sort(-1).values == want_ids.sort(-1).values).all(-1)
    print(f"P={P}: {int(same.sum())}/{same.numel()} rows identical, {int(ties.sum())} near-tie rows", flush=True)
    assert bool((same | ties | (order_ties & same_set)).all())
    from streaming_sparse_amd.legacy_components import rep_operands
    want_rv = rep_operands(g.summary, P, torch.empty_like(vrep))
    assert torch.equal(vrep.view(torch.int16), want_rv.view(torch.int16))
    tiles = [0, 17, 40, 71]
    want = ref.selected_attention(x.q, x.k, x.v, x.summary, x.basis, got, tiles=tiles).bfloat16()
    rows = torch.cat([torch.arange(t * 64, (t + 1) * 64) for t in tiles])
    check_out(out[:, rows], want[:, rows], "P=504 tiles")


def dense_ids(own, pages):
    h, t = own.shape
    rest = torch.arange(pages)
    return torch.stack([torch.cat([own[a, b:b + 1], rest[rest != own[a, b]]]) for a in range(h)
                        for b in range(t)]).reshape(h, t, pages).int()


@pytest.mark.parametrize("single", [False, True])
@pytest.mark.parametrize("all_pages", [False, True])
def test_attention_all_pages_equals_dense(device, all_pages, single):
    """Every page exact: no compensation, equals softmax attention; through
    the two-block kernel (all_pages: the caller states the table lists every
    page once) and through the table walk."""
    x = call_inputs(0, 9, heads=2)
    g = x.to(device)
    ids = dense_ids(x.own, x.pages)
    out = attention(g.q, g.k, g.v, g.summary, g.basis, ids.to(device), Workspace(), all_pages=all_pages,
                    single_av=single)
    torch.cuda.synchronize()
    want = ref.dense_attention(x.q, x.k, x.v).bfloat16()
    check_out(out, want, f"all pages exact all_pages={all_pages} single={single}")


@pytest.mark.parametrize("single", [False, True])
def test_attention_dense_432_tiles(device, single):
    """The dense call at full size (432 pages, 12 heads, the two-block
    kernel) against dense softmax attention on 8 spread query blocks."""
    x = call_inputs(1, 18)
    g = x.to(device)
    ids = dense_ids(x.own, x.pages)
    out = attention(g.q, g.k, g.v, g.summary, g.basis, ids.to(device), Workspace(), all_pages=True,
                    single_av=single)
    torch.cuda.synchronize()
    rows = tile_rows(TILES8)
    want = ref.dense_attention(x.q[:, rows], x.k, x.v).bfloat16()
    check_out(out[:, rows], want, f"dense 432 tiles single={single}")


def test_attention_padding_and_duplicates(device):
    """LUT entries outside [0, P) are not read (RV/ops.py:115): a table with
    -1 and out-of-window entries gives bit for bit the output of the table
    without them (the kernel walks the same units).  A full-length table with
    a page listed twice (so another page is missing) is walked as given
    without the all-pages flag: the repeated page counts twice and the
    missing one is compensated, as the oracle's table walk does."""
    x = call_inputs(0, 9)
    g = x.to(device)
    P = x.pages
    ids = ref.select_base(oracle_risk(x), x.own, 32)
    short = ids[..., :27]
    junk = torch.tensor([-1, P, -1000, 4096, -1], dtype=torch.int32).expand(12, 72, 5)
    padded = torch.cat([short[..., :3], junk[..., :2], short[..., 3:], junk[..., 2:]], -1).contiguous()
    ws = Workspace()
    a = attention(g.q, g.k, g.v, g.summary, g.basis, short.to(device), ws).clone()
    b = attention(g.q, g.k, g.v, g.summary, g.basis, padded.to(device), ws).clone()
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    want = ref.selected_attention(x.q, x.k, x.v, x.summary, x.basis, padded).bfloat16()
    check_out(b, want, "padded table")
    x2 = call_inputs(0, 9, heads=2)
    g2 = x2.to(device)
    dup = dense_ids(x2.own, P)
    dup[:, :, 5] = dup[:, :, 6]            # page at slot 5 missing, slot 6's page twice
    out = attention(g2.q, g2.k, g2.v, g2.summary, g2.basis, dup.to(device), Workspace())
    torch.cuda.synchronize()
    want2 = ref.selected_attention(x2.q, x2.k, x2.v, x2.summary, x2.basis, dup).bfloat16()
    check_out(out, want2, "duplicate page, full-length table")


def test_risk_checks_z(device):
    """risk() takes the reference's precomputed logits z: z of the same
    probes passes and gives the same risk as z=None; z of other probes is
    rejected."""
    x = call_inputs(0, 9)
    g = x.to(device)
    pr = ref.probes(g.q)
    z = ref.route_logits(pr.cpu(), x.summary.keys).to(device)
    a = risk_fn(pr, None, g.summary, g.theta)
    b = risk_fn(pr, z, g.summary, g.theta)
    assert torch.equal(a, b)
    with pytest.raises(ValueError):
        risk_fn(pr, z.flip(1), g.summary, g.theta)


def route_intersection_check(x, g, a, n, tag):
    """GPU intersection router vs. the oracle's quota mask and LUT; rows with
    a near tie at a partition boundary are exempt from equality."""
    P = x.pages
    cur_a = a if P != 72 else None
    ids, mask, risk, _ = route(g.q, g.summary, g.theta, tier='intersection', own=g.own, current_slots=cur_a, n=n)
    r64 = ref.risk(ref.probes(x.q), ref.route_logits(ref.probes(x.q), x.summary.keys, torch.float64),
                   x.summary.stats, x.theta, dtype=torch.float64)
    rel = float(((risk.cpu().double() - r64).abs() / r64.abs().clamp_min(1e-30)).max())
    assert rel < 1e-4, rel
    want_mask = ref.quota_mask(r64, x.own, a, n)
    want = ref.lut(r64, want_mask, x.own, 24 + n)
    ties = torch.zeros(x.own.shape, dtype=torch.bool)
    if P == 72:
        cur = r64.clone()
        cur[..., :24] = -math.inf
        cur.scatter_(-1, x.own.long()[..., None], math.inf)
        cur[..., :24] = -math.inf
        ties |= ref.near_tie_rows(cur, torch.full(x.own.shape, n))
    else:
        hist = r64.clone()
        hist[..., :24] = -math.inf
        hist[..., P - 72:] = -math.inf
        cur = r64.clone()
        cur[..., :P - 72] = -math.inf
        cur.scatter_(-1, x.own.long()[..., None], math.inf)
        ties |= ref.near_tie_rows(hist, (n - a).clamp_min(0)[:, None].expand_as(x.own))
        ties |= ref.near_tie_rows(cur, a.clamp(0, 72)[:, None].expand_as(x.own))
    got_mask = mask.cpu()
    got = ids.cpu()
    same = (got_mask == want_mask).all(-1)
    print(f"{tag}: {int(same.sum())}/{same.numel()} masks identical, {int(ties.sum())} near-tie rows", flush=True)
    assert bool((same | ties).all())
    rows = same & ~ties
    # same entries (own first, then the selection by risk, -1 padding); the
    # order among near-equal risks may differ
    assert (got[..., 0] == x.own).all()
    assert torch.equal(got[rows].sort(-1).values, want[rows].sort(-1).values)
    return got, got_mask


def test_route_intersection_first_chunk(device):
    """72-page window: the anchor frame is the chunk's first frame
    (VB/graph.py:143-148); anchors plus the top n of pages 24..71, own forced
    (own pages 0..23 are anchors themselves)."""
    x = call_inputs(2, 3)
    assert x.pages == 72
    g = x.to(device)
    ids, mask = route_intersection_check(x, g, torch.zeros(12, dtype=torch.int64), 20, "P=72")
    assert ids.shape == (12, 72, 44) and bool((mask[..., :24]).all())
    assert (mask.sum(-1) == 44).all()


def test_route_intersection_clamped_quotas(device):
    """Quotas outside their partitions at P=216: A = 0 (own not selected,
    still first in the table, the lowest selected page falls off), A = 72
    and A > 72 (the whole current frame), A + B larger than the history
    (the history is kept whole, the table padded with -1)."""
    x = call_inputs(0, 9)
    g = x.to(device)
    a = torch.tensor([0, 1, 72, 80, 30, 5, 0, 72, 40, 3, 60, 10])
    got, mask = route_intersection_check(x, g, a, 150, "clamped quotas")
    assert (mask[:, :, 24:216 - 72].sum(-1) <= 120).all()
    # heads whose quotas select fewer pages than the table holds end in -1
    padded, full = [0, 1, 3, 5, 6, 9, 11], [2, 4, 7, 8, 10]
    assert bool((got[padded] == -1).any(-1).all()) and not bool((got[full] == -1).any())
    assert bool((~mask[[0, 6]].gather(-1, x.own[[0, 6]].long()[..., None])).all())   # A = 0: own not selected


@pytest.mark.parametrize("n", [128, 192])
def test_attention_odd_window_and_slab(device, n):
    """Window of 100 pages (last rep tile partly beyond P) inside a 128-page
    summary slab, head-major strided K/V, single-page LUT; random page tables
    per block, for an even and an odd number of query blocks, up to every page."""
    h, p, cap = 3, 100, 128
    gen = torch.Generator().manual_seed(77)
    q = torch.randn(1, n, h, 128, generator=gen).bfloat16()
    kk = torch.randn(h, 64 * p, 128, generator=gen).bfloat16()
    vv = torch.randn(h, 64 * p, 128, generator=gen).bfloat16()
    basis = workload.pca_basis(vv.float().reshape(h, p, 64, 128))
    s = workload.kmeans_summaries(kk.reshape(h, p, 64, 128), vv.reshape(h, p, 64, 128), basis,
                                  torch.Generator().manual_seed(5))
    slab = Summary(*(torch.zeros((h, cap) + getattr(s, f).shape[2:], dtype=torch.bfloat16) for f in Summary.FIELDS))
    for f in Summary.FIELDS:
        getattr(slab, f)[:, :p] = getattr(s, f)
    k4 = kk.transpose(0, 1)[None]          # [1, L, H, D] view of head-major storage
    v4 = vv.transpose(0, 1)[None]
    for count in (1, 7, p):     # p: every page exact (an odd block count takes the one-block kernel)
        t = n // 64
        ids = torch.stack([torch.randperm(p, generator=gen)[:count] for _ in range(h * t)]).reshape(h, t, count).int()
        sd = slab.slice(0, p)
        gd = Summary(*(getattr(slab, f).to(device) for f in Summary.FIELDS)).slice(0, p)
        kd = kk.to(device).transpose(0, 1)[None]
        vd = vv.to(device).transpose(0, 1)[None]
        out = attention(q.to(device), kd, vd, gd, basis.to(device), ids.to(device), Workspace())
        torch.cuda.synchronize()
        want = ref.selected_attention(q, k4.contiguous(), v4.contiguous(), sd, basis, ids).bfloat16()
        check_out(out, want, f"odd window n={n} count={count}")


@pytest.mark.parametrize("single", [False, True])
def test_attention_split_pieces(device, single):
    """The last round of tiles as two pieces each (the 96 tiles past the
    last multiple of the CU count at 12 x 72 tiles on a 256-CU device,
    heads 10-11) merged by the second kernel: within the bar of the oracle
    on blocks of split and whole tiles, within 1e-3 rel-L2 of the same call
    run whole, and bit-identical over repeated calls."""
    x = call_inputs(1, 18)
    g = x.to(device)
    ws = Workspace()
    ids, _, _, _ = route(g.q, g.summary, g.theta, tier='base', own=g.own, workspace=ws)
    a = attention(g.q, g.k, g.v, g.summary, g.basis, ids, ws, single_av=single).clone()
    b = attention(g.q, g.k, g.v, g.summary, g.basis, ids, ws, single_av=single).clone()
    whole = attention(g.q, g.k, g.v, g.summary, g.basis, ids, ws, single_av=single, split=False).clone()
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    err = ref.rel_l2(a.float().cpu(), whole.float().cpu())
    print(f"split vs whole rel-L2 {err:.3e}", flush=True)
    assert err <= 1e-3, err
    tiles = [3, 50, 71]
    want = ref.selected_attention(x.q, x.k, x.v, x.summary, x.basis, ids.cpu(), tiles=tiles).bfloat16()
    rows = torch.cat([torch.arange(t * 64, (t + 1) * 64) for t in tiles])
    check_out(a[:, rows], want[:, rows], f"split pieces single={single}")


def test_attention_split_short_lists(device):
    """Unit lists shorter than two pieces: a 16-page window with one query
    block per head, so every tile is split; a table of padding only (one rep
    tile, no exact page: the first piece is empty) and a one-page table (one
    exact page and one rep tile)."""
    h, p = 2, 16
    gen = torch.Generator().manual_seed(91)
    q = torch.randn(1, 64, h, 128, generator=gen).bfloat16()
    k = torch.randn(1, 64 * p, h, 128, generator=gen).bfloat16()
    v = torch.randn(1, 64 * p, h, 128, generator=gen).bfloat16()
    vp = v[0].transpose(0, 1).reshape(h, p, 64, 128)
    basis = workload.pca_basis(vp.float())
    s = workload.kmeans_summaries(k[0].transpose(0, 1).reshape(h, p, 64, 128), vp, basis,
                                  torch.Generator().manual_seed(6))
    gd = Summary(*(getattr(s, f).to(device) for f in Summary.FIELDS))
    for table in (torch.full((h, 1, 1), -1, dtype=torch.int32), torch.tensor([[[5]], [[11]]], dtype=torch.int32)):
        out = attention(q.to(device), k.to(device), v.to(device), gd, basis.to(device), table.to(device), Workspace())
        torch.cuda.synchronize()
        want = ref.selected_attention(q, k, v, s, basis, table).bfloat16()
        check_out(out, want, f"short list {table.flatten().tolist()}")


@pytest.mark.parametrize("blocks", [256, 257])
def test_attention_split_boundary(device, blocks):
    """Tile counts at the CU-count boundary (256 CUs): 256 tiles run whole,
    257 split only the last tile into two pieces; both match the oracle on
    the first, a middle and the last tiles."""
    h, p = 1, 100
    gen = torch.Generator().manual_seed(blocks)
    n = 64 * blocks
    q = torch.randn(1, n, h, 128, generator=gen).bfloat16()
    k = torch.randn(1, 64 * p, h, 128, generator=gen).bfloat16()
    v = torch.randn(1, 64 * p, h, 128, generator=gen).bfloat16()
    vp = v[0].transpose(0, 1).reshape(h, p, 64, 128)
    basis = workload.pca_basis(vp.float())
    s = workload.kmeans_summaries(k[0].transpose(0, 1).reshape(h, p, 64, 128), vp, basis,
                                  torch.Generator().manual_seed(8))
    gd = Summary(*(getattr(s, f).to(device) for f in Summary.FIELDS))
    ids = torch.stack([torch.randperm(p, generator=gen)[:15] for _ in range(blocks)]).reshape(h, blocks, 15).int()
    out = attention(q.to(device), k.to(device), v.to(device), gd, basis.to(device), ids.to(device), Workspace())
    torch.cuda.synchronize()
    tiles = [0, blocks // 2, blocks - 1]
    want = ref.selected_attention(q, k, v, s, basis, ids, tiles=tiles).bfloat16()
    rows = torch.cat([torch.arange(t * 64, (t + 1) * 64) for t in tiles])
    check_out(out[:, rows], want[:, rows], f"{blocks} tiles")


@pytest.mark.parametrize("single", [False, True])
def test_attention_staged(device, single):
    """A staged call (the exact pages of every tile in one launch, the
    compensation's rep tiles in a second, then the merge): within the bar of
    the oracle at 432 pages on 8 spread blocks, close to the fused call
    (two-term: 1e-3 rel-L2; single-term 4e-3: each rounds its probabilities
    to one bf16 term relative to its own running maximum, which differs
    between the stages and the fused walk), and bit-identical over repeated
    calls."""
    x = call_inputs(1, 18)
    g = x.to(device)
    ws = Workspace()
    ids, _, _, _ = route(g.q, g.summary, g.theta, tier='base', own=g.own, workspace=ws)
    a = attention(g.q, g.k, g.v, g.summary, g.basis, ids, ws, single_av=single, staged=True).clone()
    b = attention(g.q, g.k, g.v, g.summary, g.basis, ids, ws, single_av=single, staged=True).clone()
    fused = attention(g.q, g.k, g.v, g.summary, g.basis, ids, ws, single_av=single).clone()
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    err = ref.rel_l2(a.float().cpu(), fused.float().cpu())
    print(f"staged vs fused rel-L2 {err:.3e}", flush=True)
    assert err <= (4e-3 if single else 1e-3), err
    want = ref.selected_attention(x.q, x.k, x.v, x.summary, x.basis, ids.cpu(), tiles=TILES8).bfloat16()
    rows = tile_rows(TILES8)
    check_out(a[:, rows], want[:, rows], f"staged single={single}")


def test_attention_staged_empty_stages(device):
    """Staged calls whose one stage has no unit: a table of every page of a
    16-page window (no rep tile: the compensation launch hands on an empty
    state) and a table of padding only (no exact page)."""
    h, p = 2, 16
    gen = torch.Generator().manual_seed(93)
    q = torch.randn(1, 128, h, 128, generator=gen).bfloat16()
    k = torch.randn(1, 64 * p, h, 128, generator=gen).bfloat16()
    v = torch.randn(1, 64 * p, h, 128, generator=gen).bfloat16()
    vp = v[0].transpose(0, 1).reshape(h, p, 64, 128)
    basis = workload.pca_basis(vp.float())
    s = workload.kmeans_summaries(k[0].transpose(0, 1).reshape(h, p, 64, 128), vp, basis,
                                  torch.Generator().manual_seed(7))
    gd = Summary(*(getattr(s, f).to(device) for f in Summary.FIELDS))
    every = torch.stack([torch.randperm(p, generator=gen) for _ in range(2 * h)]).reshape(h, 2, p).int()
    for name, table in (("every page", every), ("padding only", torch.full((h, 2, 3), -1, dtype=torch.int32))):
        out = attention(q.to(device), k.to(device), v.to(device), gd, basis.to(device), table.to(device),
                        Workspace(), staged=True)
        torch.cuda.synchronize()
        want = ref.selected_attention(q, k, v, s, basis, table).bfloat16()
        check_out(out, want, f"staged, {name}")


def _expected_ties(r, x, tier, a=None, n=None, eps=1e-3):
    """The rows a near-tie report lists, from the router's own fp32 risk with
    the same arithmetic as the kernel (|a - c| <= eps max(|a|, |c|) in fp32)
    at each selection boundary of the tier (oracle.reference.near_tie_rows on
    the partition's candidates)."""
    P = r.shape[-1]
    own = x.own
    if tier == 'base':
        cand = r.clone()
        cand[..., :24] = -math.inf
        cand.scatter_(-1, own[..., None].long(), -math.inf)
        return ref.near_tie_rows(cand, torch.full(own.shape, P * 15 // 100 - 25), rel=eps)
    nh = (n - a).clamp(0, P - 96)[:, None].expand_as(own)
    hist = r.clone()
    hist[..., :24] = -math.inf
    hist[..., P - 72:] = -math.inf
    cur = r.clone()
    cur[..., :P - 72] = -math.inf
    cur.scatter_(-1, own[..., None].long(), math.inf)
    ac = a[:, None].expand_as(own)
    return (ref.near_tie_rows(hist, nh, rel=eps) & (nh >= 1)) | (ref.near_tie_rows(cur, ac, rel=eps) & (ac >= 2))


@pytest.mark.parametrize("cfg,frames,tier", [(0, 9, 'base'), (2, 18, 'intersection')])
def test_route_reports_near_ties(device, cfg, frames, tier):
    """The router's near-tie report (the compacted row list + count of the
    reference's select_close): exactly the rows whose selection boundary
    holds two risks within 1e-3 relative, at the 216-page base call and the
    432-page intersection call; the same rows (up to rounding of risks right
    at the threshold) against the float64 oracle risk."""
    x = call_inputs(cfg, frames)
    g = x.to(device)
    H, T = 12, 72
    rows = torch.full((H * T,), -1, dtype=torch.int32, device=device)
    cnt = torch.full((1,), 12345, dtype=torch.int32, device=device)
    kw, a, n = {}, None, None
    if tier == 'intersection':
        tab = workload.quota_table(2)
        a = tab[0, 3, :, 0]
        n = int(tab[0, 3, 0].sum())
        kw = dict(current_slots=a.to(device), n=n)
    ids, _, risk, _ = route(g.q, g.summary, g.theta, tier=tier, own=g.own, ties=(rows, cnt), tie_eps=1e-3, **kw)
    torch.cuda.synchronize()
    k = int(cnt.item())
    got = rows[:k].cpu().sort().values
    assert k <= H * T and got.unique().numel() == k and bool((rows[k:] == -1).all())
    want = _expected_ties(risk.cpu(), x, tier, a, n).flatten().nonzero()[:, 0].int()
    r64 = oracle_risk(x).double()
    want64 = _expected_ties(r64, x, tier, a, n).flatten()
    print(f"{tier}: {k} near-tie rows of {H * T}; float64 oracle risk flags {int(want64.sum())}, "
          f"{int((want64[got.long()]).sum())} of them listed", flush=True)
    assert torch.equal(got, want)
    assert int((want64 != torch.zeros(H * T, dtype=torch.bool).index_fill_(0, got.long(), True)).sum()) <= \
        max(2, k // 10)
