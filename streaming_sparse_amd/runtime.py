"""Per-chunk driver of the page-sparse attention path over a stack of layers.

Mirrors the attention part of the reference's streaming runtime
(local_experiments/video_runtime_v1/runtime.py:169-350,
reproduction/vbench_current/queue_policy.py:11-56) for one 3-frame chunk:

* 4 denoise steps; per step and layer one attention call over the layer's
  resident window of P pages:
  - layer 0 is dense (runtime.py:209-211), run by the same fused kernel with
    every page exact;
  - layers 1.. refresh the current chunk's 72 page summaries (runtime.py:213-227),
    route with the intersection quotas of their (step, layer) (graph.py:150-151),
    correct the scheduled heads with Full_Pset at the scheduled (layer, step)
    (runtime.py:228, graph.py:169-208), then attend;
* the clean commit pass: every layer dense again, then the new 72 pages'
  summaries and, on Full_Pset layers, their encodings (runtime.py:328-370;
  pages stay chronological).

The K/V window of each layer is resident in HBM; each (step, layer) call gets
its own queries.  Timings cover the attention-path kernels only (no QKV
projection, cache writes or window roll).
"""
from __future__ import annotations

import math
import time
from dataclasses import dataclass, field

import torch

from . import pset, summary, workload
from .attention import Workspace
from .legacy_components import attention, rep_values
from .ops import Summary
from .route import route

ANCHORS = 24
CURRENT = 72
PSET_LAYERS = (3, 4, 5, 8, 14, 17, 27)
PSET_HEADS = (3, 4, 9)
PSET_STEPS = (0,)


@dataclass
class Layer:
    k: torch.Tensor
    v: torch.Tensor
    summary: Summary
    basis: torch.Tensor
    encoding: pset.Encoding | None = None


@dataclass
class ChunkConfig:
    layers: int = 30
    frames: int = 18
    heads: int = 12
    steps: int = 4
    seed: int = 4
    pset_layers: tuple = PSET_LAYERS
    pset_heads: tuple = PSET_HEADS
    pset_steps: tuple = PSET_STEPS
    quota_mean: float = 40.8


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


class ChunkRuntime:
    """Resident state of every layer plus the per-(step, layer) queries of
    one chunk, all generated on the device from seeds."""

    def __init__(self, cfg: ChunkConfig, device, reader_weights=None):
        self.cfg = cfg
        dev = torch.device(device)
        self.device = dev
        self.P = cfg.frames * workload.PAGES_PER_FRAME
        self.H = cfg.heads
        self.N = workload.QUERY_FRAMES * workload.TOKENS_PER_FRAME
        self.T = self.N // 64
        P, H, D = self.P, self.H, workload.HEAD_DIM
        freqs = workload.rope_table(D).to(torch.complex64).to(dev)
        g = torch.Generator(device=dev).manual_seed(workload.seed_for(cfg.seed))
        self.reader = pset.Reader(reader_weights or workload.reader_weights(cfg.seed), dev)
        self.ws = Workspace()
        self.layers = []
        for layer in range(cfg.layers):
            k = _rope_on_device(torch.randn(64 * P, H, D, generator=g, device=dev), 0, freqs)
            v = torch.randn(64 * P, H, D, generator=g, device=dev)
            k = k.to(torch.bfloat16)[None].contiguous()
            v = v.to(torch.bfloat16)[None].contiguous()
            # contiguous bf16 once here, so no call of the chunk copies it
            basis = workload.pca_basis(v[0].transpose(0, 1).reshape(H, P, 64, D).float()).to(torch.bfloat16).contiguous()
            slab = Summary(torch.empty(H, P, 4, D, device=dev, dtype=torch.bfloat16),
                           torch.empty(H, P, D, device=dev, dtype=torch.bfloat16),
                           torch.empty(H, P, 3, 8, device=dev, dtype=torch.bfloat16),
                           torch.empty(H, P, 4, 12, device=dev, dtype=torch.bfloat16))
            init = workload.kmeans_init(H, P, torch.Generator().manual_seed(workload.seed_for(cfg.seed, layer, 0, 1)))
            summary.build(k, v, basis, init.to(dev), slab, 0, P)
            enc = pset.encode(slab, basis, self.reader) if layer in cfg.pset_layers else None
            self.layers.append(Layer(k, v, slab, basis, enc))
        self.q = [[_rope_on_device(torch.randn(self.N, H, D, generator=g, device=dev), cfg.frames - 3, freqs)
                   .to(torch.bfloat16)[None].contiguous() for _ in range(cfg.layers)] for _ in range(cfg.steps + 1)]
        self.init_current = workload.kmeans_init(H, CURRENT, torch.Generator().manual_seed(
            workload.seed_for(cfg.seed, 0, 0, 9))).to(device=dev, dtype=torch.int32)
        quotas = workload.quota_table(cfg.seed, layers=max(cfg.layers - 1, 1), steps=cfg.steps, heads=H,
                                      mean_total=cfg.quota_mean)
        self.quota_a = quotas[..., 0].to(torch.int32).to(dev)           # [steps, layers-1, H]
        self.quota_n = quotas[..., 0, :].sum(-1).tolist()                # [steps][layers-1]
        self.theta = torch.tensor([1.0, 1.0, 1.0, 0.5], device=dev).expand(H, 4).contiguous()
        self.lse = torch.empty(H, self.T, 16, device=dev)
        own = torch.arange(self.T, device=dev) + P - self.T
        rest = torch.arange(P, device=dev)
        dense = torch.cat([own[:, None], rest[None].expand(self.T, -1)], 1)
        keep = dense != own[:, None]
        keep[:, 0] = True
        self.dense_ids = dense[keep].reshape(self.T, P)[None].expand(H, -1, -1).to(torch.int32).contiguous()

    def dense_call(self, layer: int, q):
        L = self.layers[layer]
        return attention(q, L.k, L.v, L.summary, L.basis, self.dense_ids, self.ws, all_pages=True)

    def sparse_call(self, layer: int, step: int, q):
        """One sparse attention call (layers >= 1): current summaries,
        encodings when Full_Pset is scheduled, route (+ correction), attend."""
        cfg, L, P = self.cfg, self.layers[layer], self.P
        correct = layer in cfg.pset_layers and step in cfg.pset_steps
        summary.build(L.k, L.v, L.basis, self.init_current, L.summary, P - CURRENT, CURRENT)
        if correct:
            pset.encode(L.summary, L.basis, self.reader, out=L.encoding, first=P - CURRENT, pages=CURRENT)
        a = self.quota_a[step, layer - 1]
        n = int(self.quota_n[step][layer - 1])
        vrep = self.ws.tensor('rt_rep_values', (L.summary.mean.shape[0], P, 4, 128), q.device, torch.bfloat16)
        ids, _, _, stats = route(q, L.summary, self.theta, tier='intersection', current_slots=a, n=n,
                                 workspace=self.ws, want_mask=correct, lse_out=self.lse if correct else None,
                                 full_pset=cfg.pset_heads if correct else None, encoding=L.encoding,
                                 reader=self.reader, rep_basis=L.basis, rep_out=vrep)
        return attention(q, L.k, L.v, L.summary, L.basis, ids, self.ws, rep_values=vrep)

    def commit(self, layer: int, q):
        """Clean step: dense attention, then the new pages' summaries (and
        encodings on Full_Pset layers)."""
        out = self.dense_call(layer, q)
        L, P = self.layers[layer], self.P
        summary.build(L.k, L.v, L.basis, self.init_current, L.summary, P - CURRENT, CURRENT)
        if L.encoding is not None:
            pset.encode(L.summary, L.basis, self.reader, out=L.encoding, first=P - CURRENT, pages=CURRENT)
        return out

    def run_chunk(self):
        for step in range(self.cfg.steps):
            for layer in range(self.cfg.layers):
                q = self.q[step][layer]
                if layer == 0:
                    self.dense_call(layer, q)
                else:
                    self.sparse_call(layer, step, q)
        for layer in range(self.cfg.layers):
            self.commit(layer, self.q[self.cfg.steps][layer])

    def run_dense_chunk(self, sdpa=False):
        """The dense baseline: every call of the chunk dense (our kernel with
        all pages exact, or torch's scaled_dot_product_attention)."""
        for step in range(self.cfg.steps + 1):
            for layer in range(self.cfg.layers):
                q = self.q[step][layer]
                if sdpa:
                    L = self.layers[layer]
                    torch.nn.functional.scaled_dot_product_attention(
                        q[0].transpose(0, 1)[None], L.k[0].transpose(0, 1)[None], L.v[0].transpose(0, 1)[None])
                else:
                    self.dense_call(layer, q)

    def calls_per_chunk(self):
        cfg = self.cfg
        sparse = cfg.steps * (cfg.layers - 1)
        return dict(sparse=sparse, dense=cfg.steps + cfg.layers,
                    full_pset=len([l for l in cfg.pset_layers if l < cfg.layers]) * len(cfg.pset_steps))
