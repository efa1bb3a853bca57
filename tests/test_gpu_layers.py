"""The layer-batched entries (one launch over several layers) against one
call per layer, bit for bit: ssa_summary_layers, ssa_encode_layers,
ssa_anchor_rebase_layers and ssa_commit_pages_layers, on three layers of
different caches, bases and orders (one layer in token order)."""
import pytest
import torch

from streaming_sparse_amd import _lib, pset, summary, workload
from streaming_sparse_amd.legacy_components import HEAD_DIM, kv_strides
from streaming_sparse_amd.ops import Summary

pytestmark = pytest.mark.gpu

H, P, NL = 12, 432, 3


def same(a, b):
    return torch.equal(a.view(torch.uint8), b.view(torch.uint8))


def caches(device, seed):
    g = torch.Generator(device=device).manual_seed(seed)
    mk = lambda: torch.randn(1, 64 * P, H, HEAD_DIM, generator=g, device=device).to(torch.bfloat16)
    return [(mk(), mk()) for _ in range(NL)]


def bases(device):
    out = []
    for l in range(NL):
        sample = torch.randn(H, 24, 64, HEAD_DIM, generator=torch.Generator().manual_seed(40 + l))
        out.append(workload.pca_basis(sample).to(torch.bfloat16).to(device).contiguous())
    return out


def slab(device):
    return Summary(torch.zeros(H, P, 4, HEAD_DIM, device=device, dtype=torch.bfloat16),
                   torch.zeros(H, P, HEAD_DIM, device=device, dtype=torch.bfloat16),
                   torch.zeros(H, P, 3, 8, device=device, dtype=torch.bfloat16),
                   torch.zeros(H, P, 4, 12, device=device, dtype=torch.bfloat16))


@pytest.mark.parametrize("first,pages", [(360, 72), (0, 24)])
def test_summary_and_encode_layers(device, first, pages):
    kv = caches(device, 3)
    bs = bases(device)
    init_all = workload.kmeans_init(H, 72, torch.Generator().manual_seed(5)).to(device=device, dtype=torch.int32)
    init = init_all[:, :pages]                      # a slice, as the anchor refresh passes it
    one = [slab(device) for _ in range(NL)]
    many = [slab(device) for _ in range(NL)]
    for (k, v), b, s in zip(kv, bs, one):
        summary.build(k, v, b, init, s, first, pages)
    summary.build_layers([k for k, _ in kv], [v for _, v in kv], bs, init, many, first, pages)
    reader = pset.Reader(workload.reader_weights(0), device)
    enc_one = [pset.Encoding.empty(H, P, device) for _ in range(NL)]
    enc_many = [pset.Encoding.empty(H, P, device) for _ in range(NL)]
    for s, b, e in zip(one, bs, enc_one):
        pset.encode(s, b, reader, out=e, first=first, pages=pages)
    pset.encode_layers(many, bs, reader, enc_many, first, pages)
    torch.cuda.synchronize()
    for a, b in zip(one, many):
        assert all(same(getattr(a, f), getattr(b, f)) for f in Summary.FIELDS)
        assert bool(getattr(a, 'mean')[:, first:first + pages].abs().sum() > 0)
    for a, b in zip(enc_one, enc_many):
        assert same(a.coef, b.coef) and same(a.mean, b.mean) and same(a.detail, b.detail)
        assert bool(a.coef[:, first:first + pages].float().abs().sum() > 0)


def test_anchor_rebase_and_commit_layers(device):
    L = _lib.lib()
    stream = _lib.stream_handle(device)
    kv = caches(device, 7)
    tok, head = kv_strides(*kv[0])
    g = torch.Generator(device=device).manual_seed(11)
    canon = [torch.randn(1536, H, HEAD_DIM, generator=g, device=device).to(torch.bfloat16) for _ in range(NL)]
    phase = torch.randn(32, 2, generator=g, device=device, dtype=torch.float64)
    one = [k.clone() for k, _ in kv]
    many = [k.clone() for k, _ in kv]
    for c, d in zip(canon, one):
        _lib.check(L.ssa_anchor_rebase(_lib.ptr(c), H * HEAD_DIM, HEAD_DIM, _lib.ptr(d), tok, head, _lib.ptr(phase), 32,
                                       1536, H, stream), "ssa_anchor_rebase")
    _lib.check(L.ssa_anchor_rebase_layers(NL, _lib.ptrs(canon), H * HEAD_DIM, HEAD_DIM, _lib.ptrs(many), tok, head,
                                          _lib.ptr(phase), 32, 1536, H, stream), "ssa_anchor_rebase_layers")
    torch.cuda.synchronize()
    assert all(same(a, b) for a, b in zip(one, many))
    assert not same(one[0], kv[0][0])
    # commit: chunk K/V [4608, H, 128] per layer, orders per layer (layer 1 in token order), slots wrapping the ring
    src_k = [torch.randn(4608, H, HEAD_DIM, generator=g, device=device).to(torch.bfloat16) for _ in range(NL)]
    src_v = [torch.randn(4608, H, HEAD_DIM, generator=g, device=device).to(torch.bfloat16) for _ in range(NL)]
    orders = [torch.stack([torch.randperm(4608, generator=torch.Generator().manual_seed(20 + 13 * l + h))
                           for h in range(H)]).to(device=device, dtype=torch.int32) for l in range(NL)]
    orders[1] = None
    slots = torch.tensor(list(range(400, 432)) + list(range(24, 64)), dtype=torch.int32, device=device)
    ko, vo = [k.clone() for k, _ in kv], [v.clone() for _, v in kv]
    km, vm = [k.clone() for k, _ in kv], [v.clone() for _, v in kv]
    for l in range(NL):
        _lib.check(L.ssa_commit_pages(_lib.ptr(src_k[l]), _lib.ptr(src_v[l]), H * HEAD_DIM, HEAD_DIM,
                                      _lib.ptr(orders[l]), 72, _lib.ptr(slots), P, _lib.ptr(ko[l]), _lib.ptr(vo[l]),
                                      tok, head, H, stream), "ssa_commit_pages")
    _lib.check(L.ssa_commit_pages_layers(NL, _lib.ptrs(src_k), _lib.ptrs(src_v), H * HEAD_DIM, HEAD_DIM,
                                         _lib.ptrs(orders), 72, _lib.ptr(slots), P, _lib.ptrs(km), _lib.ptrs(vm), tok,
                                         head, H, stream), "ssa_commit_pages_layers")
    torch.cuda.synchronize()
    assert all(same(a, b) for a, b in zip(ko, km)) and all(same(a, b) for a, b in zip(vo, vm))
    assert not same(ko[0], kv[0][0])
