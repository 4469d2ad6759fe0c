"""The C ABI library loads and exports every symbol declared in include/*.h (CPU only)."""

import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    names = []
    for header in sorted((ROOT / "include").glob("*.h")):
        text = header.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"\b(spr_\w+)\s*\(", text)
    return sorted(set(names))


def test_header_declares_entry_points():
    names = declared_symbols()
    assert "spr_last_error" in names and len(names) >= 10


def test_library_exports_every_declared_symbol():
    from sparsepr_amd import _lib

    if not _lib.LIB_PATH.exists():
        pytest.fail(f"{_lib.LIB_PATH} is not built (run __graft_entry__.build())")
    lib = _lib.load()  # also binds every signature in _lib.SIGNATURES
    for name in declared_symbols():
        assert hasattr(lib, name), f"{name} missing from {_lib.LIB_PATH.name}"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert lib.spr_abi_version() == 2
    assert isinstance(lib.spr_last_error(), bytes)


def test_entry_points_validate_arguments_without_a_gpu():
    """Argument checks run on the host before any launch, so they work here."""
    from sparsepr_amd import _lib

    lib = _lib.load()
    # bad k for the label sort
    st = lib.spr_argsort_labels(None, 1, 10, 0, None, None, None, None, 0, None)
    assert st == 1 and b"k=0" in lib.spr_last_error()
    # unsupported head dim for the bf16 assign
    st = lib.spr_kmeans_assign_bf16(16, 16, 16, None, 0, None, 1, 10, 4, 96, 16, None)
    assert st == 1 and b"head dim 96" in lib.spr_last_error()
    # empty problems are no-ops
    assert lib.spr_permute_rows(None, None, None, 0, 5, 256, None) == 0
    # the attention takes the row maximum before scaling, so the scale must be positive
    for scale in (0.0, -0.125, float("inf")):
        st = lib.spr_block_sparse_attention_run(None, None, None, None, 0, 0, 1, 0, 128, 1, 1, scale, None, None,
                                                None, None, None)
        assert st == 1 and b"scale must be positive" in lib.spr_last_error()
        st = lib.spr_dense_attention(None, None, None, 0, 1, 1, 16, 128, scale, 1, None, 0, None, None, 0, None)
        assert st == 1 and b"scale must be positive" in lib.spr_last_error()
