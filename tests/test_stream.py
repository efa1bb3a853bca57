"""Host logic of the rolling window (CPU): the ring of history pages against
slot sequences worked out by hand from RV/runtime.py:38-46, the anchor
rebase schedule, and the oracle's anchor rebase against the closed form of
RoPE (a rebased frame-0 key is the key rotated at the shifted frame)."""
import torch

from oracle import reference as ref
from streaming_sparse_amd import workload
from streaming_sparse_amd.runtime import PageRing, rebase_offset, runs


def test_ring_slots_full_window():
    """history 360, sink 24: chunks 0..4 fill pages 0..359 in order; chunk 5
    (the first whose window is full) overwrites pages 24..95, chunk 6 pages
    96..167; page 0..23 (the anchor frame) is never written again."""
    r = PageRing(360, 24)
    seen = []
    for c in range(12):
        slots = r.commit_slots()
        assert len(set(slots)) == 72
        seen.append(slots)
        r.commit()
    for c in range(5):
        assert seen[c] == list(range(72 * c, 72 * c + 72))
    assert seen[5] == list(range(24, 96)) and seen[6] == list(range(96, 168))
    assert all(min(s) >= 24 for s in seen[1:])
    assert r.n == 360 and r.commits == 12
    # FIFO over [24, 360): each commit after the window fills overwrites the oldest pages
    assert seen[9] == list(range(312, 360)) + list(range(24, 48))


def test_ring_slots_wrap_small():
    """history 168, sink 24: the third commit wraps: 144..167 then 24..71."""
    r = PageRing(168, 24)
    got = []
    for c in range(4):
        got.append((r.n, r.commit_slots()))
        r.commit()
    assert [n for n, _ in got] == [0, 72, 144, 168]
    assert got[2][1] == list(range(144, 168)) + list(range(24, 72))
    assert got[3][1] == list(range(72, 144))
    assert runs(got[2][1]) == [(144, 24, 0), (24, 48, 24)]
    assert runs(list(range(5, 77))) == [(5, 72, 0)]


def test_ring_without_sink():
    r = PageRing(216, 0)
    for _ in range(3):
        r.commit()
    assert r.commit_slots() == list(range(72)) and r.n == 216


def test_rebase_schedule():
    """The anchor is rebased from chunk 6 on by 3c - 15 frames, so the
    current frames 3c..3c+2 stay 15..17 frames from it."""
    assert [rebase_offset(c) for c in range(9)] == [0, 0, 0, 0, 0, 0, 3, 6, 9]
    for c in range(6, 20):
        assert [3 * c + i - rebase_offset(c) for i in range(3)] == [15, 16, 17]


def test_shift_temporal_closed_form():
    """Shifting a frame-0 RoPE'd key by `o` frames equals RoPE at frame `o`
    (temporal pairs), leaves the spatial pairs and the rows past `tokens`
    untouched, and is the identity at offset 0."""
    g = torch.Generator().manual_seed(3)
    freqs = workload.rope_table(128)
    x = torch.randn(1536 * 2, 2, 128, generator=g, dtype=torch.float64)
    at0 = workload.apply_rope(x, 0, freqs)[None]          # frames 0 and 1, float64
    for o in (3, 9, 40):
        got = ref.shift_temporal(at0, 1536, freqs, o)
        want = workload.apply_rope(x[:1536], o, freqs)
        torch.testing.assert_close(got[0, :1536, :, :44], want[:, :, :44], rtol=0, atol=1e-12)
        assert torch.equal(got[0, :1536, :, 44:], at0[0, :1536, :, 44:])
        assert torch.equal(got[0, 1536:], at0[0, 1536:])
    assert torch.equal(ref.shift_temporal(at0, 1536, freqs, 0), at0)
