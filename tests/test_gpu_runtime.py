"""The per-chunk driver (streaming_sparse_amd.runtime) on a small stack:
3 layers, 216-page window, Full_Pset on layer 1 at step 0.  Checks each kind
of call against the oracle on the driver's own state: the dense layer (all
pages exact) against softmax attention, a corrected sparse call against
SelectedAttention.fixed on the page table it used, and the recomputed
current-page summaries against the summary oracle."""
import pytest
import torch

from oracle import reference as ref
from oracle import summary as osum
from streaming_sparse_amd.ops import Summary
from streaming_sparse_amd.runtime import ChunkConfig, ChunkRuntime

pytestmark = pytest.mark.gpu
REL_L2, MAX_ABS = 5e-3, 2e-2


def _check(got, want, tag):
    g, w = got.detach().cpu().float(), want.float()
    err = ref.rel_l2(g, w)
    mx = float((g - w).abs().max())
    print(f"{tag}: rel-L2 {err:.3e} max-abs {mx:.3e}", flush=True)
    assert err <= REL_L2 and mx <= MAX_ABS, (tag, err, mx)


def test_chunk_driver_calls(device):
    cfg = ChunkConfig(layers=3, frames=9, pset_layers=(1,), seed=6)
    rt = ChunkRuntime(cfg, device)
    rt.run_chunk()
    torch.cuda.synchronize()
    L0, L1 = rt.layers[0], rt.layers[1]
    P = rt.P
    # dense layer: every page exact == softmax attention (2 heads on the CPU)
    q0 = rt.q[0][0]
    out0 = rt.dense_call(0, q0).clone()
    torch.cuda.synchronize()
    hs = [0, 7]
    want0 = ref.dense_attention(q0[:, :, hs].cpu(), L0.k[:, :, hs].cpu(), L0.v[:, :, hs].cpu()).bfloat16()
    _check(out0[:, :, hs], want0, "dense layer")
    # corrected sparse call of layer 1, step 0: oracle attention on its page table
    q1 = rt.q[0][1]
    out1 = rt.sparse_call(1, 0, q1).clone()
    ids = rt.ws.entries[('route_ids', (12, rt.T, 24 + int(rt.quota_n[0][0])), torch.device(device),
                         torch.int32)].cpu()
    torch.cuda.synchronize()
    s_cpu = Summary(*(getattr(L1.summary, f).cpu() for f in Summary.FIELDS))
    want1 = ref.selected_attention(q1.cpu(), L1.k.cpu(), L1.v.cpu(), s_cpu, L1.basis.cpu().float(), ids)
    _check(out1, want1.bfloat16(), "sparse layer with Full_Pset")
    assert (ids[..., 0] == torch.arange(rt.T) + P - 72).all()
    # the driver's current-page summaries are the summary oracle's
    kp = L1.k[0].transpose(0, 1).reshape(12, P, 64, 128)[:, P - 72:].cpu()
    vp = L1.v[0].transpose(0, 1).reshape(12, P, 64, 128)[:, P - 72:].cpu()
    want = osum.summaries(kp, vp, L1.basis.cpu().float(), rt.init_current.cpu())
    ok = want['margin'] > 1e-5
    for name in ('keys', 'mean'):
        got = getattr(s_cpu, name)[:, P - 72:].float()[ok]
        w = want[name].float()[ok]
        assert bool(((got - w).abs() <= w.abs() * 2.0 ** -7 + 1e-6).all()), name
    calls = rt.calls_per_chunk()
    assert calls == dict(sparse=8, dense=7, full_pset=1)
