"""The full streaming workload at its real size, through size-independent
properties (the oracle would take hours here): 30 layers x 12 heads, 4
denoise steps + the clean step, a 360-page history ring (432-page window),
Full_Pset on layers {3,4,5,8,14,17,27} x heads {3,4,9} at step 0.

Two runtimes built from the same seed run chunks 0..6 (the window fills at
chunk 5; chunk 6 runs after the ring wrapped and the anchor was rebased):
* every call of chunk 6 (150 of them) gives bit-identical outputs in both,
  and so do their ring and summary state afterwards (no atomics or
  order-dependent reductions anywhere on the path);
* the call counts are the workload's: 116 sparse calls (7 with Full_Pset)
  and 34 dense ones per full-window chunk;
* every output is finite."""
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
