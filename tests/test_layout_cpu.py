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


def test_plan_8bit_transposed_b():
    """An int8 B given as a transposed view (a weight kept [N][K]) runs K-major, unscaled
    (int32 C) or W8A8; with a block that has no K-major form it is copied row-major."""
    bt = _t((64, 304), "int8")[:, :300].t()      # [300][64] view, columns 304 bytes apart
    a = txdot.aligned_rows(_t((16, 300), "int8"), col_ok=False)
    for c, sm in ((tx.I32, tx.SCALE_NONE), (tx.BF16, tx.SCALE_ROWCOL)):
        assert txdot._b_kmajor_ok(a, bt, c, sm, (0, 0, 0), 0)
        assert txdot.aligned_rows(bt, col_ok=True) is bt
        p = txdot.plan_for(a, bt, c, sm)
        assert p.desc.flags & tx.FLAG_B_KMAJOR and p.desc.ldb == 304
    assert not txdot._b_kmajor_ok(a, bt, tx.BF16, tx.SCALE_ROWCOL, (256, 224, 128), 0)
    b = txdot.aligned_rows(bt, col_ok=False)
    assert b.stride(1) == 1 and b.shape == (300, 64)
    p = txdot.plan_for(a, b, tx.BF16, tx.SCALE_ROWCOL, block=(256, 224, 128))
    assert not p.desc.flags & tx.FLAG_B_KMAJOR


@pytest.mark.parametrize("dtype_name,txt,M,tile,other", [
    ("int8", tx.I32, 16, (16, 128, 128), (256, 224, 128)),
    ("int8", tx.I32, 600, (256, 256, 128), (256, 224, 128)),
    ("bfloat16", tx.F32, 16, (16, 64, 128), (128, 128, 64)),
    ("bfloat16", tx.F32, 100, (256, 256, 64), (64, 64, 32))])
def test_transposed_b_with_an_explicit_block(dtype_name, txt, M, tile, other):
    """K-major B where the tile has that form: the planner's own choice, or that tile asked
    for by name; another block copies B row-major (dot) or is refused (plan_for)."""
    bt = _t((64, 304), dtype_name)[:, :300].t()
    a = txdot.aligned_rows(_t((M, 300), dtype_name), col_ok=False)
    for blk in ((0, 0, 0), tile):
        assert txdot._b_kmajor_ok(a, bt, txt, tx.SCALE_NONE, blk, 0)
        p = txdot.plan_for(a, bt, txt, block=blk)
        assert p.desc.flags & tx.FLAG_B_KMAJOR and (p.desc.block_m, p.desc.block_n,
                                                    p.desc.block_k) == tile
    assert not txdot._b_kmajor_ok(a, bt, txt, tx.SCALE_NONE, other, 0)
    b = txdot.aligned_rows(bt, col_ok=False)
    assert b.stride(1) == 1
    assert not txdot.plan_for(a, b, txt, block=other).desc.flags & tx.FLAG_B_KMAJOR
    with pytest.raises(ValueError, match="transposed view"):
        txdot.plan_for(a, bt, txt, block=other)


def test_plan_rejects_a_transposed_a():
    a = _t((64, 64)).t()[:, :32]          # columns contiguous: A must be row-major
    with pytest.raises(ValueError):
        txdot.plan_for(a, _t((32, 16)), tx.F32)
