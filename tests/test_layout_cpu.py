"""How the binding reads a 2-D view's layout (dot.py `_layout`, `aligned_rows`,
`plan_for`), on CPU tensors: row-major, a transposed view of row-major storage
(K-major B), and the stride of a size-1 dimension, which says nothing about
the layout.  Planning runs on the host; nothing here launches."""
import importlib

import pytest

import triton_ext_amd as tx

txdot = importlib.import_module("triton_ext_amd.dot")  # the module (the package exports dot())


def _t(shape, dtype_name="bfloat16"):
    import torch
    return torch.zeros(shape, dtype=getattr(torch, dtype_name))


def test_layout_kinds():
    import torch
    st = _t((220, 8))                     # [N][K'] storage, rows 16 bytes apart
    assert txdot._layout(st[:, :5]) == ("row", 8)
    assert txdot._layout(st[:, :5].t()) == ("col", 8)       # K-major B, K = 5
    assert txdot._layout(st[:, :1].t()) == ("col", 8)       # K = 1: one row, elements 8 apart
    assert txdot._layout(_t((1, 300)).t()) == ("col", 300)  # N = 1, adjacent elements: K-major
    assert txdot._layout(_t((1, 300)).t(), col_ok=False) == ("row", 1)  # or one row-major column
    assert txdot._layout(st[:, :5].t(), col_ok=False)[0] is None
    assert txdot._layout(_t((64, 64))[::2, ::2])[0] is None  # neither rows nor columns contiguous
    assert txdot._layout(torch.zeros(1, 1)) == ("row", 1)


def test_plan_k1_kmajor_b():
    """q @ k.T with one head dim: B = k.t() is [1, N] with elements ldk apart."""
    a = txdot.aligned_rows(_t((5, 8))[:, :1])
    b = _t((220, 8))[:, :1].t()
    assert txdot.aligned_rows(b) is b     # already 16-byte columns
    p = txdot.plan_for(a, b, tx.F32)
    assert p.desc.flags & tx.FLAG_B_KMAJOR and p.desc.ldb == 8 and p.desc.K == 1


@pytest.mark.parametrize("dtype_name,txt", [("int8", tx.I32), ("bfloat16", tx.F32)])
def test_plan_single_column_b(dtype_name, txt):
    """N = 1, B = x.t() for x [1, K]: row-major (any dtype), after the copy into
    16-byte rows that its 1-element pitch needs."""
    K = 300
    a = txdot.aligned_rows(_t((40, K), dtype_name))
    b = txdot.aligned_rows(_t((1, K), dtype_name).t(), col_ok=False)
    assert b.shape == (K, 1) and (b.stride(0) * b.element_size()) % 16 == 0
    p = txdot.plan_for(a, b, txt, ldc=4)  # C rows of one 4-byte element, 16 bytes apart
    assert not p.desc.flags & tx.FLAG_B_KMAJOR and p.desc.N == 1


def test_plan_8bit_transposed_b_is_copied_row_major():
    """An int8 B given as a transposed view (no K-major 8-bit kernel) is copied row-major."""
    b = txdot.aligned_rows(_t((64, 300), "int8").t(), col_ok=txdot._b_col_ok(_t((1, 1), "int8")))
    assert b.stride(1) == 1 and b.shape == (300, 64)
    p = txdot.plan_for(txdot.aligned_rows(_t((16, 300), "int8"), col_ok=False), b, tx.I32)
    assert not p.desc.flags & tx.FLAG_B_KMAJOR


def test_plan_rejects_a_transposed_a():
    a = _t((64, 64)).t()[:, :32]          # columns contiguous: A must be row-major
    with pytest.raises(ValueError):
        txdot.plan_for(a, _t((32, 16)), tx.F32)
