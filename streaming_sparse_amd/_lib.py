"""ctypes binding of libssattn.so (declared in include/ssattn.h).

The library is built in-tree by ``streaming_sparse_amd.build``.  There is no
fallback: if the library is missing or a call fails, an error is raised.
"""
from __future__ import annotations

import ctypes
import os

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libssattn.so")
_lib = None

_vp, _i, _ll, _f = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong, ctypes.c_float
# return type of the entry points that do not return a status
RESTYPES = {"ssa_attention_workspace_bytes": _ll}
SIGNATURES = {
    "ssa_route_stamps": [_vp, _ll],
    "ssa_attn_stamps": [_vp, _ll],
    "ssa_rep_operands": [_vp, _vp, _i, _i, _i, _i, _vp],
    "ssa_attention": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _ll, _ll, _i, _vp, _ll,
                      _vp],
    "ssa_attention_workspace_bytes": [_i, _i, _i, _i, _i],
    "ssa_route": [_vp, _ll, _ll, _ll, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i,
                  _vp, _vp, _i, _f, _vp, _vp, _vp],
    "ssa_select": [_vp, _vp, _vp, _i, _i, _f, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp],
    "ssa_encode": [_vp, _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i,
                   _i, _vp],
    "ssa_summary": [_vp, _vp, _ll, _ll, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp],
    "ssa_summary_layers": [_i, _vp, _vp, _ll, _ll, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp],
    "ssa_encode_layers": [_i, _vp, _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i,
                          _i, _i, _i, _i, _vp],
    "ssa_anchor_rebase_layers": [_i, _vp, _ll, _ll, _vp, _ll, _ll, _vp, _i, _i, _i, _vp],
    "ssa_commit_pages_layers": [_i, _vp, _vp, _ll, _ll, _vp, _i, _vp, _i, _vp, _vp, _ll, _ll, _i, _vp],
    "ssa_summary_write": [_vp, _vp, _ll, _ll, _vp, _vp, _ll, _ll, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i,
                          _vp],
    "ssa_pset": [_vp, _ll, _ll, _ll, _i, _vp, _i, _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _vp,
                 _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp],
    "ssa_anchor_rebase": [_vp, _ll, _ll, _vp, _ll, _ll, _vp, _i, _i, _i, _vp],
    "ssa_commit_pages": [_vp, _vp, _ll, _ll, _vp, _i, _vp, _i, _vp, _vp, _ll, _ll, _i, _vp],
    "ssa_group_order": [_vp, _vp, _ll, _ll, _ll, _vp, _vp, _vp, _vp, _i, _i, _i, _vp, _vp, _vp, _vp],
    "ssa_pset_noalloc": [_vp, _ll, _ll, _ll, _i, _vp, _i, _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i,
                         _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp],
}


def load(path):
    """A ctypes handle of the library at `path` with the entry points typed."""
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built; run `python -m streaming_sparse_amd.build`")
    handle = ctypes.CDLL(path)
    for name, args in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.argtypes = args
        fn.restype = RESTYPES.get(name, ctypes.c_int)
    return handle


def lib():
    global _lib
    if _lib is None:
        _lib = load(LIB_PATH)
    return _lib


def use(path):
    """Route every later call of this process through the library at `path`
    (a measurement build of the same sources, streaming_sparse_amd.build)."""
    global _lib
    _lib = load(path)
    return _lib


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def ptrs(tensors):
    """A host array of the tensors' device pointers (None -> NULL), for the
    entries that take one tensor per layer."""
    return (ctypes.c_void_p * len(tensors))(*[None if t is None else t.data_ptr() for t in tensors])


def stream_handle(device=None):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def check(status: int, name: str):
    if status != 0:
        raise RuntimeError(f"{name} failed with hipError {status}")
