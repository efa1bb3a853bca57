"""The C-ABI library loads and exports every entry point include/ssattn.h
declares, and the Python binding matches the header's arity (no GPU calls)."""
import ctypes
import os
import re

import pytest

from streaming_sparse_amd import _lib, build

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    text = open(os.path.join(ROOT, "include", "ssattn.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"\b(?:int|long long)\s+(ssa_\w+)\s*\(([^)]*)\)\s*;", text):
        out[m.group(1)] = len([a for a in m.group(2).split(",") if a.strip()])
    return out


def test_header_declares_entry_points():
    assert set(declared()) == {"ssa_rep_operands", "ssa_attention", "ssa_attention_workspace_bytes", "ssa_route", "ssa_select", "ssa_encode", "ssa_pset",
                               "ssa_summary", "ssa_summary_write", "ssa_pset_noalloc", "ssa_anchor_rebase", "ssa_commit_pages",
                               "ssa_summary_layers", "ssa_encode_layers", "ssa_anchor_rebase_layers",
                               "ssa_commit_pages_layers",
                               "ssa_group_order", "ssa_route_stamps", "ssa_attn_stamps"}


@pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH), reason="libssattn.so not built")
def test_library_exports_every_declared_symbol():
    handle = ctypes.CDLL(_lib.LIB_PATH)
    for name, nargs in declared().items():
        assert hasattr(handle, name), name
        assert len(_lib.SIGNATURES[name]) == nargs, name
    _lib.lib()


@pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH), reason="libssattn.so not built")
def test_product_library_has_no_phase_stamps():
    """The router's phase stamps and the attention kernel's step stamps exist
    only in the measurement build: the product library's ssa_route_stamps and
    ssa_attn_stamps report hipErrorNotSupported (801) without touching their
    arguments."""
    assert _lib.lib().ssa_route_stamps(None, 0) == 801
    assert _lib.lib().ssa_attn_stamps(None, 0) == 801


@pytest.mark.skipif(not os.path.exists(build.STAMPS_LIB), reason="libssattn_stamps.so not built")
def test_measurement_library_exports_every_declared_symbol():
    """The measurement build (the same sources with the router's and the
    attention kernel's stamps compiled in) exports the same entry points, so
    streaming_sparse_amd.route_phases and attn_steps can route every call
    through it."""
    handle = ctypes.CDLL(build.STAMPS_LIB)
    for name in declared():
        assert hasattr(handle, name), name

