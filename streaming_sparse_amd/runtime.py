"""Streaming driver of the page-sparse attention path over a stack of layers,
with a rolling KV window.

Mirrors the attention side of the reference's streaming runtime:
local_experiments/video_runtime_v1/runtime.py:169-370 (VideoRuntime.forward,
commit_group), local_experiments/review_v1/runtime.py:14-55 (PageStore, the
ring of history pages), reproduction/vbench_current/phase.py:4-25 with
local_experiments/anchor_rebase.py:8-18 (anchor rebase) and
reproduction/vbench_current/queue_policy.py:11-56 (quota schedule).

Each layer keeps a resident K/V cache of history_pages + 72 pages and a
summary slab of the same capacity.  A 3-frame chunk of 72 pages runs:

* from chunk 6 on (the window is full), the anchor rebase: the first frame's
  keys (24 pages, never overwritten) are re-rotated from their state after
  chunk 0's commit so that the current frames sit 15..17 frames from the
  anchor (offset 3c - 15, VB history/*/video.py), and the anchor pages'
  summaries (and Full_Pset encodings) are rebuilt from them (VB/phase.py);
* 4 denoise steps and the clean step; at each, every layer gets the chunk's
  K/V written after its n valid history pages (pages [n, n + 72)) and runs one
  attention call over the window of P = n + 72 pages:
  - dense (every page exact, the same fused kernel) for layer 0, for the
    clean step and while the history holds at most 72 pages
    (runtime.py:209-211); the reference runs these through its ordinary
    dense attention (engine.dense), whose P.V is one bf16 product, so they
    run single-term here too;
  - otherwise the current pages' summaries are rebuilt, Full_Pset encodings
    too where scheduled, then the intersection router with the
    (window, step, layer) quotas, Full_Pset on the scheduled heads
    (runtime.py:213-257, graph.py:169-210), and the attention;
* the commit of the clean step, after all its calls: the chunk's tokens of
  every layer are grouped into pages in one batch (GroupingOps.group,
  RV/runtime.py:57-68; the first chunk re-sorted by frame so the anchor frame
  fills pages 0..23, runtime.py:358-363), then per layer the grouped pages
  are written into the ring slots (PageStore.commit_slots: after the first
  commit the slots wrap inside [24, history_pages), so the anchor frame
  stays), with their summaries and, on Full_Pset layers, encodings at those
  slots (runtime.py:330-370).

Q/K/V are seeded N(0, 1) with Wan RoPE at the chunk's absolute frames,
generated on the device before the chunk runs; writing K/V into the cache
stands in for the projection that writes them there in the reference.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib, group, pset, summary, workload
from .attention import Workspace
from .legacy_components import HEAD_DIM, REP_OP_ELEMS, attention, kv_strides, rep_tiles
from .ops import Summary
from .route import route

ANCHORS = 24
CURRENT = 72
ANCHOR_TOKENS = ANCHORS * 64
PSET_LAYERS = (3, 4, 5, 8, 14, 17, 27)
PSET_HEADS = (3, 4, 9)
PSET_STEPS = (0,)
TEMPORAL_PAIRS = 22          # complex RoPE pairs of the temporal axis at head_dim 128
REBASE_FROM_CHUNK = 6        # first chunk whose window is full and whose anchor is rebased


@dataclass
class StreamConfig:
    layers: int = 30
    heads: int = 12
    steps: int = 4
    history_pages: int = 360       # with the 72 current pages: a 432-page (18-frame) window
    sink_pages: int = 24           # the anchor frame, kept out of the ring's wrap
    seed: int = 4
    pset_layers: tuple = PSET_LAYERS
    pset_heads: tuple = PSET_HEADS
    pset_steps: tuple = PSET_STEPS
    quota_mean: float = 40.8
    sparse_start_chunks: tuple = ()   # chunks with <= 72 history pages that still run sparse
    grouping: bool = True             # group the committed tokens into pages (False: token order)
    # 'intersection': anchor/current/history quotas with Full_Pset (VB/queue_policy.py); 'base': the
    # base tier, own + 24 anchors + the floor(0.15 P) - 25 highest-risk pages, no swap correction
    # (VR/runtime.py:279-288; a window of at least 96 pages)
    tier: str = 'intersection'


class PageRing:
    """Ring bookkeeping of the history pages (RV/runtime.py:14-46): `n`
    valid pages, the next write page and the commit count.  The first commit
    writes pages [0, 72); later ones wrap inside [sink, history_pages)."""

    def __init__(self, history_pages: int, sink_pages: int):
        if history_pages < CURRENT + sink_pages or history_pages % 1 or sink_pages < 0:
            raise ValueError("history_pages must hold a chunk beyond the sink")
        self.history_pages = history_pages
        self.sink = sink_pages
        self.n = self.write = self.commits = 0

    def commit_slots(self) -> list:
        sink = self.sink if self.commits else 0
        span = self.history_pages - sink
        return [sink + (self.write + i - sink) % span for i in range(CURRENT)]

    def commit(self):
        end = self.write + CURRENT
        self.write = self.sink + (end - self.sink) % (self.history_pages - self.sink)
        self.n = min(self.history_pages, self.n + CURRENT)
        self.commits += 1


def runs(slots) -> list:
    """Contiguous runs (first slot, length, offset into the chunk) of a slot list."""
    out = []
    for i, s in enumerate(slots):
        if out and s == out[-1][0] + out[-1][1]:
            out[-1][1] += 1
        else:
            out.append([s, 1, i])
    return [tuple(r) for r in out]


def _batches(items, size: int = 32):
    """`items` in runs of at most `size` (the layer limit of one batched
    launch)."""
    return [items[i:i + size] for i in range(0, len(items), size)]


def rebase_offset(chunk: int) -> int:
    """Temporal shift of the anchor frame for a chunk (0 before the window is full)."""
    return 3 * chunk - 15 if chunk >= REBASE_FROM_CHUNK else 0


def _rope_on_device(x, first_frame, freqs):
    """Wan RoPE (wan/modules/causal_model.py:27-55) on a [L, H, D] fp32 device
    tensor at frames first_frame + i // 1536."""
    L, H, D = x.shape
    c = D // 2
    ct, ch = c - 2 * (c // 3), c // 3
    frames = L // workload.TOKENS_PER_FRAME
    ft, fh, fw = freqs.split([ct, ch, ch], dim=1)
    gh, gw = workload.GRID_H, workload.GRID_W
    f = torch.cat([
        ft[first_frame:first_frame + frames].view(frames, 1, 1, -1).expand(frames, gh, gw, -1),
        fh[:gh].view(1, gh, 1, -1).expand(frames, gh, gw, -1),
        fw[:gw].view(1, 1, gw, -1).expand(frames, gh, gw, -1),
    ], dim=-1).reshape(L, 1, c)
    z = torch.view_as_complex(x.reshape(L, H, c, 2).contiguous())
    return torch.view_as_real(z * f).reshape(L, H, D)


class ChunkInputs(list):
    """[steps + 1][layers] of (q, k, v), plus the clean step's K/V of all
    layers as [L, N, H, D] blocks (clean_k, clean_v) whose per-layer views
    are the clean step's entries."""


@dataclass
class Layer:
    k: torch.Tensor             # [1, 64 (history + 72), H, 128] bf16 resident cache
    v: torch.Tensor
    slab: Summary               # [H, history + 72, ...]
    basis: torch.Tensor         # [H, 128, 8] bf16
    encoding: pset.Encoding | None = None
    canonical: torch.Tensor | None = None   # anchor keys after chunk 0's commit [1536, H, 128] bf16


class StreamRuntime:
    """Resident per-layer state of a stream of 3-frame chunks."""

    def __init__(self, cfg: StreamConfig, device, reader_weights=None):
        if cfg.tier not in ('intersection', 'base'):
            raise ValueError(f"unknown tier {cfg.tier!r}")
        self.cfg = cfg
        dev = torch.device(device)
        self.device = dev
        H, D = cfg.heads, HEAD_DIM
        self.H = H
        self.cap = cfg.history_pages + CURRENT
        self.N = CURRENT * 64
        self.T = CURRENT
        self.ring = PageRing(cfg.history_pages, cfg.sink_pages)
        self.chunk = 0
        self.freqs = workload.rope_table(D)                      # complex128, CPU
        self.freqs_dev = self.freqs.to(torch.complex64).to(dev)
        self.reader = pset.Reader(reader_weights or workload.reader_weights(cfg.seed), dev)
        self.ws = Workspace()
        self.layers = []
        for layer in range(cfg.layers):
            g = torch.Generator().manual_seed(workload.seed_for(cfg.seed, layer, 0, 2))
            sample = torch.randn(H, ANCHORS, 64, D, generator=g)
            basis = workload.pca_basis(sample).to(torch.bfloat16).to(dev).contiguous()
            k = torch.zeros(1, 64 * self.cap, H, D, device=dev, dtype=torch.bfloat16)
            v = torch.zeros_like(k)
            slab = Summary(torch.zeros(H, self.cap, 4, D, device=dev, dtype=torch.bfloat16),
                           torch.zeros(H, self.cap, D, device=dev, dtype=torch.bfloat16),
                           torch.zeros(H, self.cap, 3, 8, device=dev, dtype=torch.bfloat16),
                           torch.zeros(H, self.cap, 4, 12, device=dev, dtype=torch.bfloat16))
            enc = pset.Encoding.empty(H, self.cap, dev) if layer in cfg.pset_layers else None
            self.layers.append(Layer(k, v, slab, basis, enc))
        self.init = workload.kmeans_init(H, CURRENT, torch.Generator().manual_seed(
            workload.seed_for(cfg.seed, 0, 0, 9))).to(device=dev, dtype=torch.int32).contiguous()
        self.theta = torch.tensor([1.0, 1.0, 1.0, 0.5], device=dev).expand(H, 4).contiguous()
        self.lse = torch.empty(H, self.T, 16, device=dev)
        self.group_weights = group.GroupWeights.seeded(cfg.layers, H, cfg.seed, dev) if cfg.grouping else None
        self.page_dst = group.page_destinations(cfg.history_pages)
        self.last_order = None
        self.record = None            # a list to collect a copy of every call's output, or None
        self.own = None
        self.quotas = {}
        self.last = {}                # ids / out of the most recent call, for inspection
        self.calls = dict(sparse=0, dense=0, full_pset=0)

    # ------------------------------------------------------------- inputs --

    def chunk_inputs(self, chunk: int | None = None):
        """Seeded Q/K/V of every (step, layer) of a chunk, RoPE at its absolute
        frames 3c..3c+2: list [steps + 1][layers] of (q [1,N,H,D], k, v
        [N,H,D]) bf16 device tensors.  The chunk's quota table (the policy
        table the reference loads, VB/queue_policy.py:18-33) is prepared with
        them."""
        c = self.chunk if chunk is None else chunk
        cfg = self.cfg
        dev = self.device
        self.quota(c)
        # the clean step's K/V of all layers in one [L, N, H, D] block each, so
        # the commit groups every layer in one batch
        clean_k = torch.empty(cfg.layers, self.N, self.H, HEAD_DIM, device=dev, dtype=torch.bfloat16)
        clean_v = torch.empty_like(clean_k)
        out = []
        for step in range(cfg.steps + 1):
            row = []
            for layer in range(cfg.layers):
                g = torch.Generator(device=dev).manual_seed(
                    workload.seed_for(cfg.seed, layer, step, 1000 + 3 * c))
                q, k, v = (torch.randn(self.N, self.H, HEAD_DIM, generator=g, device=dev) for _ in range(3))
                q = _rope_on_device(q, 3 * c, self.freqs_dev).to(torch.bfloat16)[None].contiguous()
                k = _rope_on_device(k, 3 * c, self.freqs_dev).to(torch.bfloat16)
                if step == cfg.steps:
                    clean_k[layer].copy_(k)
                    clean_v[layer].copy_(v)
                    k, v = clean_k[layer], clean_v[layer]
                else:
                    k, v = k.contiguous(), v.to(torch.bfloat16).contiguous()
                row.append((q, k, v))
            out.append(row)
        out = ChunkInputs(out)
        out.clean_k, out.clean_v = clean_k, clean_v
        return out

    def quota(self, chunk: int):
        """(A [steps, layers-1, H] int32 on the device, A+B per (step, layer)
        as host ints) of a chunk.  Chunks 0 and 1 (windows of 72 and 144
        pages, sparse only when listed in sparse_start_chunks) take the
        reference's fixed quotas n = 4 / 12 with A = 4 / 7 for every call
        (VB/queue_policy.py:25-28); later chunks a seeded table."""
        if chunk not in self.quotas:
            for done in [c for c in self.quotas if c < chunk - 1]:
                del self.quotas[done]
            if chunk < 2:
                a, n = (4, 7)[chunk], (4, 12)[chunk]
                tab = torch.empty(self.cfg.steps, max(self.cfg.layers - 1, 1), self.H, 2, dtype=torch.int64)
                tab[..., 0] = a
                tab[..., 1] = n - a
            else:
                tab = workload.quota_table(self.cfg.seed, layers=max(self.cfg.layers - 1, 1), steps=self.cfg.steps,
                                           heads=self.H, mean_total=self.cfg.quota_mean, window=chunk)
            # pinned staging: the copy does not wait for the stream's earlier work
            cur = tab[..., 0].to(torch.int32).pin_memory().to(self.device, non_blocking=True)
            self.quotas[chunk] = (cur, tab[..., 0, :].sum(-1).tolist())
        return self.quotas[chunk]

    # ------------------------------------------------------------ chunk ----

    def begin_chunk(self):
        """The chunk's commit slots on the device, and the anchor rebase from
        the window-full chunk on (VB/phase.py:4-25)."""
        c = self.chunk
        self.slots = self.ring.commit_slots()
        key = ('rt_slots', (CURRENT,), self.device, torch.int32)
        if key not in self.ws.entries:
            self.ws.entries[key] = torch.empty(CURRENT, device=self.device, dtype=torch.int32)
        self.slots_dev = self.ws.entries[key]
        self.slots_dev.copy_(torch.tensor(self.slots, dtype=torch.int32, pin_memory=True), non_blocking=True)
        if c >= REBASE_FROM_CHUNK:
            self.rebase_anchor(rebase_offset(c))

    def rebase_anchor(self, offset: int):
        """Anchor keys of every layer = the chunk-0 anchor keys with the
        temporal RoPE pairs shifted by `offset` frames; the anchor pages'
        summaries and encodings rebuilt from them.  Each of the three steps
        runs every layer in one launch (the reference loops over the layers,
        VB/phase.py:4-25)."""
        ph = self.freqs[offset, :TEMPORAL_PAIRS]
        phase = torch.view_as_real(ph).to(torch.float64).contiguous().pin_memory().to(self.device, non_blocking=True)
        H = self.H
        for group_ in _batches(self.layers):
            tok, head = kv_strides(group_[0].k, group_[0].v)
            _lib.check(_lib.lib().ssa_anchor_rebase_layers(
                len(group_), _lib.ptrs([L.canonical for L in group_]), H * HEAD_DIM, HEAD_DIM,
                _lib.ptrs([L.k for L in group_]), tok, head, _lib.ptr(phase), TEMPORAL_PAIRS, ANCHOR_TOKENS, H,
                _lib.stream_handle(self.device)), "ssa_anchor_rebase_layers")
        self._summarise(0, ANCHORS, self.init[:, :ANCHORS])

    def dense_window(self, chunk: int | None = None) -> bool:
        n = self.ring.n
        c = self.chunk if chunk is None else chunk
        return n <= CURRENT and c not in self.cfg.sparse_start_chunks

    def layer_call(self, step: int, layer: int, q, k, v):
        """One attention call of the current chunk: the chunk's K/V written into
        the window (a sparse call writes them in the pass of its current-page
        summaries), then a dense or sparse call (the clean step's commits
        follow all its calls, see commit_chunk)."""
        cfg, L = self.cfg, self.layers[layer]
        n = self.ring.n
        P = n + CURRENT
        tok0 = 64 * n
        kw = L.k[:, :64 * P]
        vw = L.v[:, :64 * P]
        s = L.slab.slice(0, P)
        clean = step == cfg.steps
        if clean or layer == 0 or self.dense_window():
            L.k[0, tok0:tok0 + self.N].copy_(k)
            L.v[0, tok0:tok0 + self.N].copy_(v)
            out = attention(q, kw, vw, s, L.basis, self.dense_ids(P), self.ws, all_pages=True, single_av=True)
            self.calls['dense'] += 1
        else:
            out = self.sparse_call(step, layer, q, kw, vw, P, (k, v))
        self.last = dict(step=step, layer=layer, pages=P, out=out)
        if self.record is not None:
            self.record.append(out.clone())
        return out

    def sparse_call(self, step, layer, q, kw, vw, P, src):
        cfg, L = self.cfg, self.layers[layer]
        correct = cfg.tier == 'intersection' and L.encoding is not None and step in cfg.pset_steps
        summary.build(L.k, L.v, L.basis, self.init, L.slab, P - CURRENT, CURRENT, src=src)
        s = L.slab.slice(0, P)
        ops = self.ws.tensor('rt_rep_ops', (self.H, rep_tiles(P), REP_OP_ELEMS), q.device, torch.bfloat16)
        if cfg.tier == 'base':
            ids, _, _, _ = route(q, s, self.theta, tier='base', workspace=self.ws, want_mask=False, rep_out=ops)
            self.calls['sparse'] += 1
            self.last_ids = ids
            return attention(q, kw, vw, s, L.basis, ids, self.ws, rep_ops=ops)
        if correct:
            pset.encode(L.slab, L.basis, self.reader, out=L.encoding, first=P - CURRENT, pages=CURRENT)
        a_tab, n_tab = self.quota(self.chunk)
        a = a_tab[step, layer - 1]
        n = int(n_tab[step][layer - 1])
        ids, _, _, _ = route(q, s, self.theta, tier='intersection', current_slots=a, n=n, workspace=self.ws,
                             want_mask=correct, lse_out=self.lse if correct else None,
                             full_pset=cfg.pset_heads if correct else None, encoding=L.encoding,
                             reader=self.reader, rep_out=ops)
        self.calls['sparse'] += 1
        self.calls['full_pset'] += int(correct)
        self.last_ids = ids
        return attention(q, kw, vw, s, L.basis, ids, self.ws, rep_ops=ops)

    def commit_chunk(self, inputs):
        """The clean step's commit of every layer: one batched grouping of the
        chunk's tokens (the first chunk re-sorted by frame so the anchor frame
        fills pages 0..23), then the grouped pages of every layer into the
        ring slots (tokens in `order[layer]` [H, 4608], None: token order)
        with their summaries and encodings (VR/runtime.py:356-370), each step
        over all layers in one launch."""
        order = None
        if self.cfg.grouping:
            order = group.order(inputs.clean_k, inputs.clean_v, self.group_weights, first_chunk=self.chunk == 0,
                                page_dst=self.page_dst, workspace=self.ws)
        self.last_order = order
        for group_ in _batches(list(range(self.cfg.layers))):
            Ls = [self.layers[layer] for layer in group_]
            tok, head = kv_strides(Ls[0].k, Ls[0].v)
            ks = [inputs.clean_k[layer] for layer in group_]
            vs = [inputs.clean_v[layer] for layer in group_]
            src_tok, src_head = ks[0].stride(0), ks[0].stride(1)
            orders = [None if order is None else order[layer] for layer in group_]
            _lib.check(_lib.lib().ssa_commit_pages_layers(
                len(group_), _lib.ptrs(ks), _lib.ptrs(vs), src_tok, src_head, _lib.ptrs(orders), CURRENT,
                _lib.ptr(self.slots_dev), self.cap, _lib.ptrs([L.k for L in Ls]), _lib.ptrs([L.v for L in Ls]), tok,
                head, self.H, _lib.stream_handle(self.device)), "ssa_commit_pages_layers")
        for first, length, off in runs(self.slots):
            self._summarise(first, length, self.init[:, off:off + length])

    def _summarise(self, first: int, length: int, init):
        """Summaries of pages [first, first + length) of every layer, and the
        encodings of the Full_Pset layers, each in one launch per 32 layers."""
        for group_ in _batches(self.layers):
            summary.build_layers([L.k for L in group_], [L.v for L in group_], [L.basis for L in group_], init,
                                 [L.slab for L in group_], first, length)
        encoded = [L for L in self.layers if L.encoding is not None]
        for group_ in _batches(encoded):
            pset.encode_layers([L.slab for L in group_], [L.basis for L in group_], self.reader,
                               [L.encoding for L in group_], first, length)

    def end_chunk(self):
        if self.chunk == 0:
            for L in self.layers:
                L.canonical = L.k[0, :ANCHOR_TOKENS].clone()
        self.ring.commit()
        self.chunk += 1

    def run_chunk(self, inputs):
        self.begin_chunk()
        for step in range(self.cfg.steps + 1):
            for layer in range(self.cfg.layers):
                q, k, v = inputs[step][layer]
                self.layer_call(step, layer, q, k, v)
        self.commit_chunk(inputs)
        self.end_chunk()

    def run_dense_chunk(self, inputs, sdpa=False):
        """The same chunk's calls, every one dense over the window (this
        library's kernel with every page exact, or torch's
        scaled_dot_product_attention); the ring is not advanced."""
        n = self.ring.n
        P = n + CURRENT
        for step in range(self.cfg.steps + 1):
            for layer in range(self.cfg.layers):
                q, k, v = inputs[step][layer]
                L = self.layers[layer]
                L.k[0, 64 * n:64 * n + self.N].copy_(k)
                L.v[0, 64 * n:64 * n + self.N].copy_(v)
                kw, vw = L.k[:, :64 * P], L.v[:, :64 * P]
                if sdpa:
                    torch.nn.functional.scaled_dot_product_attention(
                        q[0].transpose(0, 1)[None], kw[0].transpose(0, 1)[None], vw[0].transpose(0, 1)[None])
                else:
                    attention(q, kw, vw, L.slab.slice(0, P), L.basis, self.dense_ids(P), self.ws, all_pages=True,
                              single_av=True)

    def dense_ids(self, P: int):
        """Every page of a P-page window per block, own page (P - 72 + t) first."""
        key = ('rt_dense_ids', (self.H, self.T, P), self.device, torch.int32)
        if key not in self.ws.entries:
            own = torch.arange(self.T) + P - self.T
            rest = torch.arange(P)
            ids = torch.cat([own[:, None], rest[None].expand(self.T, -1)], 1)
            keep = ids != own[:, None]
            keep[:, 0] = True
            self.ws.entries[key] = ids[keep].reshape(self.T, P)[None].expand(self.H, -1, -1).to(
                device=self.device, dtype=torch.int32).contiguous()
        return self.ws.entries[key]

    def calls_per_chunk(self):
        cfg = self.cfg
        dense_window = self.dense_window()
        sparse = 0 if dense_window else cfg.steps * (cfg.layers - 1)
        return dict(sparse=sparse, dense=cfg.steps * cfg.layers + cfg.layers - sparse,
                    full_pset=0 if dense_window or cfg.tier != 'intersection' else
                    len([l for l in cfg.pset_layers if 0 < l < cfg.layers]) * len(cfg.pset_steps))
