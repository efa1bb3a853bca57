"""Workspace buffer cache, as local_experiments/video_runtime_v1/attention.py:7-13.

Buffers are keyed by (name, shape, device, dtype) and reused across calls, so a
returned output tensor is overwritten by the next call with the same key.
"""
from __future__ import annotations

import torch


class Workspace:
    def __init__(self):
        self.entries = {}

    def tensor(self, name, shape, device, dtype):
        key = (name, tuple(shape), torch.device(device), dtype)
        if key not in self.entries:
            self.entries[key] = torch.empty(shape, device=device, dtype=dtype)
        return self.entries[key]

    def bytes(self):
        return sum(x.numel() * x.element_size() for x in self.entries.values())
