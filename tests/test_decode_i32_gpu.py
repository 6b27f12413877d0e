"""The decode kernels' int32 sums, read directly.

An unscaled int8 -> int32 tt.dot of decode shape (small M, HBM-bound) runs on
the W8A8 decode kernels (decode_i8.h up to M = 48, decode_rows_i8.h past it)
with an int32 epilogue, so their split-K sums are observed bit for bit, not
only through the bf16 epilogue.  The reference: the exact integer product.
The int8 operands make every partial and final sum an integer below 2^31
(127^2 * 8192 = 132,128,768), which float64 holds exactly, so a float64
BLAS product is the int64 product here.

The interpreter fixture w8a8_rowcol_rtz (tests/golden) then closes the loop
on the W8A8 epilogue: the GPU's int32 sums, scaled as the interpreter does
((float(acc) * sa) * sb in fp32) and truncated to bf16 as the interpreter's
cast does (T:runtime/interpreter.py:461-467), give the fixture's bytes
exactly.  The GPU's own W8A8 epilogue rounds to nearest even instead (as
compiled Triton does); it is held to the oracle's RNE mode elsewhere.
"""
import os

import numpy as np
import pytest

import oracle
import triton_ext_amd as tx
from dotcase import from_device, say, to_device, uniform_i8

pytestmark = pytest.mark.gpu


def exact(a, b):
    return (a.astype(np.float64) @ b.astype(np.float64)).astype(np.int64)


def run_i32(gpu, a, b, acc=None, block=(0, 0, 0)):
    import torch
    M, K = a.shape
    N = b.shape[1]
    # the plan dot() makes: operand rows padded to 16 bytes
    up = lambda x, m: -(-x // m) * m
    plan = tx.plan(tx.make_desc(M, N, K, tx.I8, tx.I32, block=block, lda=up(K, 16),
                                ldb=up(N, 16), ldc=up(N, 4),
                                flags=tx.FLAG_ACCUMULATE if acc is not None else 0))
    c = tx.dot(to_device(a, gpu), to_device(b, gpu), out_dtype=torch.int32, block=block,
               acc=None if acc is None else to_device(acc, gpu))
    torch.cuda.synchronize()
    return plan, from_device(c)


@pytest.mark.parametrize("M", [1, 16, 64, 256])
def test_decode_int32_sums_exact(gpu, M):
    """BASELINE's W8A8 shapes (N = K = 8192) without the epilogue: every int32 sum."""
    N = K = 8192
    say(f"int8->int32 decode M={M} N={N} K={K}")
    a = uniform_i8((M, K), 100 + M)
    b = uniform_i8((K, N), 200 + M)
    plan, got = run_i32(gpu, a, b)
    assert plan.kernel == tx.KERNEL_DECODE_I8 and plan.split_k > 1
    want = exact(a, b)
    assert np.array_equal(got.astype(np.int64), want), \
        f"{np.count_nonzero(got != want)} sums differ"


@pytest.mark.parametrize("M,N,K", [(16, 8191, 8191), (5, 1000, 4001), (48, 4100, 2000),
                                   (100, 4100, 2000), (200, 260, 1000), (250, 304, 256),
                                   (1, 24, 64), (3, 128, 1)])
def test_decode_int32_ragged(gpu, M, N, K):
    """Ragged K and N (the masked K tail, the column quad that crosses N), both
    kernels, one and several row slices."""
    say(f"int8->int32 decode ragged M={M} N={N} K={K}")
    a = uniform_i8((M, K), M + 7)
    b = uniform_i8((K, N), N + 7)
    plan, got = run_i32(gpu, a, b)  # rows not 16 bytes apart are padded by dot()
    assert plan.kernel == tx.KERNEL_DECODE_I8
    want = exact(a, b)
    assert np.array_equal(got.astype(np.int64), want), \
        f"{np.count_nonzero(got != want)} sums differ"


def test_decode_int32_junk_padding(gpu):
    """Operands in storage whose row padding and extra rows hold random bytes: an
    unmasked element past K or N would change a sum."""
    import torch
    M, N, K = 16, 8190, 8190
    say(f"int8->int32 decode junk-padded M={M} N={N} K={K}")
    rng = np.random.default_rng(5)
    A = rng.integers(-128, 128, size=(M + 3, K + 18), dtype=np.int8)
    B = rng.integers(-128, 128, size=(K + 5, N + 2), dtype=np.int8)
    da, db = to_device(A, gpu), to_device(B, gpu)
    c = tx.dot(da[:M, :K], db[:K, :N], out_dtype=torch.int32)
    torch.cuda.synchronize()
    assert np.array_equal(from_device(c).astype(np.int64), exact(A[:M, :K], B[:K, :N]))


@pytest.mark.parametrize("M,N,K", [(16, 8192, 8192), (128, 4096, 4096), (7, 300, 100)])
def test_decode_int32_accumulate(gpu, M, N, K):
    """tl.dot(a, b, acc) with an int32 acc: C = acc + A @ B, exactly."""
    say(f"int8->int32 decode acc M={M} N={N} K={K}")
    a = uniform_i8((M, K), 31)
    b = uniform_i8((K, N), 32)
    acc = np.random.default_rng(33).integers(-2**28, 2**28, size=(M, N), dtype=np.int32)
    plan, got = run_i32(gpu, a, b, acc=acc)
    assert plan.kernel == tx.KERNEL_DECODE_I8
    assert np.array_equal(got.astype(np.int64), exact(a, b) + acc)


def test_w8a8_fixture_from_gpu_int32_sums(gpu):
    """The interpreter's W8A8 bytes from the GPU's int32 sums: scale in fp32 as
    (float(acc) * sa) * sb, truncate to bf16, as the interpreter does."""
    from test_oracle_cpu import GOLDEN, load_fixture
    f = load_fixture(os.path.join(GOLDEN, "w8a8_rowcol_rtz.npz"))
    say("w8a8_rowcol_rtz fixture through the int32 decode epilogue")
    plan, acc = run_i32(gpu, f["a"], f["b"])
    assert plan.kernel == tx.KERNEL_DECODE_I8
    assert np.array_equal(acc.astype(np.int64), exact(f["a"], f["b"]))
    v = (acc.astype(np.float32) * f["sa"][:, None]) * f["sb"][None, :]  # fp32, in order
    trunc = (v.view(np.uint32) >> 16).astype(np.uint16)
    assert np.array_equal(trunc, f["c"])
    # the RNE rounding of the same values, which the GPU's W8A8 epilogue and compiled
    # Triton use, differs from these truncated bytes by one bf16 step where it rounds up
    rne = oracle.f32_to_bf16(v, oracle.ROUND_RNE)
    d = rne.astype(np.int32) - f["c"].astype(np.int32)
    assert set(np.unique(d)) <= {0, 1, -1}
    say(f"w8a8_rowcol_rtz: {np.count_nonzero(d)} of {d.size} outputs round differently")
