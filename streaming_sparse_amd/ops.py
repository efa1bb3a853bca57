"""Host-side types of the page-sparse attention path.

``Summary`` mirrors local_experiments/review_v1/ops.py:30-37: per page of one
head, 4 representative keys, the V mean, a 3x8 Haar/rank-8 detail code and a
4x12 block of routing statistics, all bf16.  Slices ``[:, a:b]`` of larger
``[H, Pcap, ...]`` slabs are allowed; the head stride of ``mean`` gives the slab
capacity, as in local_experiments/video_runtime_v1/legacy_components.py:43.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

# Haar contrasts over the 4 representatives of a page
# (local_experiments/review_v1/ops.py:10).
HAAR = ((1, 1, -1, -1), (1, -1, 1, -1), (1, -1, -1, 1))


@dataclass
class Summary:
    keys: torch.Tensor     # [H, P, 4, D]
    mean: torch.Tensor     # [H, P, D]
    detail: torch.Tensor   # [H, P, 3, 8]
    stats: torch.Tensor    # [H, P, 4, 12]

    FIELDS = ('keys', 'mean', 'detail', 'stats')

    def bytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.keys, self.mean, self.detail, self.stats))

    def slice(self, a: int, b: int) -> "Summary":
        return Summary(*(getattr(self, n)[:, a:b] for n in self.FIELDS))

    @property
    def pages(self) -> int:
        return self.mean.shape[1]

    @property
    def head_pages(self) -> int:
        """Page capacity of the underlying slab (head stride / D)."""
        return self.mean.stride(0) // self.mean.shape[-1]
