"""loop_split planner vs brute-force enumeration of the predicate.

The reference pass (R:pass/LoopSplit/LoopSplit.cpp:125-197) turns
`for iv in [lo, hi) step s: if (iv P c) ...` into two loops with the compare
folded.  Correctness means: every iteration of the first loop has predicate
== first_value, every iteration of the second has second_value, and together
they are exactly the original iterations.  That is checked here by
enumerating iterations, for all predicates, both operand orders, and step 1
and step > 1 -- including the cases where the reference's arithmetic is wrong
(sgt/sge at step 1, step rounding when (mid - lo) % step == 0).
"""
import itertools

import pytest

import triton_ext_amd as tx

OPS = {
    tx.CMP_SLT: lambda a, b: a < b, tx.CMP_SLE: lambda a, b: a <= b,
    tx.CMP_SGT: lambda a, b: a > b, tx.CMP_SGE: lambda a, b: a >= b,
    tx.CMP_ULT: lambda a, b: a < b, tx.CMP_ULE: lambda a, b: a <= b,
    tx.CMP_UGT: lambda a, b: a > b, tx.CMP_UGE: lambda a, b: a >= b,
}


def brute_check(lo, hi, step, pred, c, rhs):
    s = tx.loop_split_plan(lo, hi, step, pred, c, iv_on_rhs=rhs, bits=64)
    assert s.split == 1
    its = list(range(lo, hi, step))
    first = list(range(lo, min(s.midp, hi), step)) if s.midp > lo else []
    second = list(range(s.midp, hi, step))
    assert first + second == its, (lo, hi, step, pred, c, rhs, s.midp)
    assert len(first) == s.first_trips and len(second) == s.second_trips
    f = OPS[pred]
    val = (lambda iv: f(c, iv)) if rhs else (lambda iv: f(iv, c))
    assert all(val(iv) == bool(s.first_value) for iv in first), (lo, hi, step, pred, c, rhs)
    assert all(val(iv) == bool(s.second_value) for iv in second), (lo, hi, step, pred, c, rhs)
    assert s.second_value == (not s.first_value)
    # the split point sits on the iteration grid (or at a bound)
    assert s.midp in (lo, hi) or (s.midp - lo) % step == 0


@pytest.mark.parametrize("pred", [tx.CMP_SLT, tx.CMP_SLE, tx.CMP_SGT, tx.CMP_SGE])
@pytest.mark.parametrize("rhs", [False, True])
def test_signed_brute_force(pred, rhs):
    for lo, hi, step in itertools.product(range(-3, 3), range(-2, 45, 3), (1, 2, 3, 10)):
        for c in range(-6, 50, 1):
            brute_check(lo, hi, step, pred, c, rhs)


@pytest.mark.parametrize("pred", [tx.CMP_ULT, tx.CMP_ULE, tx.CMP_UGT, tx.CMP_UGE])
def test_unsigned_nonnegative(pred):
    for lo, hi, step in itertools.product(range(0, 3), range(0, 30, 4), (1, 3, 10)):
        for c in range(0, 35):
            brute_check(lo, hi, step, pred, c, False)


def test_declines():
    # non-positive step (reference: failure(), LoopSplit.cpp:130-138)
    assert tx.loop_split_plan(0, 10, 0, tx.CMP_SLT, 5).split == 0
    assert tx.loop_split_plan(0, 10, -1, tx.CMP_SLT, 5).split == 0
    # eq / ne are not in CmpTypeMap (LoopSplit.cpp:35-44)
    assert tx.loop_split_plan(0, 10, 1, tx.CMP_EQ, 5).split == 0
    assert tx.loop_split_plan(0, 10, 1, tx.CMP_NE, 5).split == 0
    # unsigned compare over negative values: orders differ, decline
    assert tx.loop_split_plan(-4, 10, 1, tx.CMP_ULT, 5).split == 0
    with pytest.raises(tx.TxError):
        tx.loop_split_plan(0, 1 << 40, 1, tx.CMP_SLT, 5, bits=32)  # does not fit i32


def test_lit_cases_structure():
    """The five FileCheck cases of R:pass/LoopSplit/test/loop-split.mlir.

    Each loop is `scf.for %iv = 0 to %n step S` with `if (iv P %mid)
    {addf} else {subf}`.  The checks require: first loop subf (predicate
    false), second loop addf (true) for sgt/sge; the reverse for slt/sle.
    Split points are checked against the iteration values directly: the
    reference's arithmetic (R:pass/LoopSplit/LoopSplit.cpp:156-174) splits
    sgt/sge one iteration early at step 1 and overshoots by one step when
    (mid - lo) % step == 0, so its midp is not the oracle here."""
    n, mid = 40, 13
    for pred, first_true in ((tx.CMP_SGT, False), (tx.CMP_SGE, False),
                             (tx.CMP_SLT, True), (tx.CMP_SLE, True)):
        s = tx.loop_split_plan(0, n, 1, pred, mid)
        assert s.first_value == first_true
        brute_check(0, n, 1, pred, mid, False)
    # sgt: first iteration with iv > 13 is 14; sge: 13; slt: 13; sle: 14
    assert tx.loop_split_plan(0, n, 1, tx.CMP_SGT, mid).midp == 14
    assert tx.loop_split_plan(0, n, 1, tx.CMP_SGE, mid).midp == 13
    assert tx.loop_split_plan(0, n, 1, tx.CMP_SLT, mid).midp == 13
    assert tx.loop_split_plan(0, n, 1, tx.CMP_SLE, mid).midp == 14
    # step10 case: iv in {0,10,20,30}, iv < 13 true for 0,10 -> split at 20
    assert tx.loop_split_plan(0, n, 10, tx.CMP_SLT, 13).midp == 20
    assert tx.loop_split_plan(0, n, 10, tx.CMP_SLT, 20).midp == 20


@pytest.mark.parametrize("K,bk,split,main,tail", [
    (4096, 64, 4096, 64, 0), (4000, 64, 3968, 62, 32), (512, 32, 512, 16, 0),
    (33, 32, 32, 1, 1), (31, 32, 0, 0, 31), (0, 64, 0, 0, 0), (64, 64, 64, 1, 0),
    (8192, 128, 8192, 64, 0), (7168, 128, 7168, 56, 0), (100, 128, 0, 0, 100)])
def test_k_tail(K, bk, split, main, tail):
    """The dot's K loop: predicate `k > K - bk` marks the one masked step."""
    import ctypes
    L = tx.load("libloop_split.so")
    ks, km, kt = ctypes.c_int64(), ctypes.c_int32(), ctypes.c_int32()
    assert L.tx_loop_split_k(K, bk, ctypes.byref(ks), ctypes.byref(km), ctypes.byref(kt)) == 0
    assert (ks.value, km.value, kt.value) == (split, main, tail)
    # brute force: steps whose loads need a mask are exactly those past the split
    steps = list(range(0, K, bk))
    masked = [k for k in steps if k + bk > K]
    assert [k for k in steps if k >= split] == masked
    assert main == len(steps) - len(masked)
