"""The fp8 decode kernel (decode_f8.h) against the oracle.

fp8 dots with M <= 64 stream B once on the decode kernel: unscaled fp8
(e4m3 / e5m2 in any mix) to fp32 C, and e4m3 with 1x128 A-group and 128x128
B-block scales (the block-scaled fp8 dot) to bf16 or fp32 C.  128-column
strips, 128-row K batches (one scale block each), split-K with the fp32
partials summed in split order.  The bar is the north_star's fp bar,
|d| <= 1e-3 s + 1e-2 |ref|: s = sqrt(K) for block-scaled inputs (N(0,1) before
quantisation), s = sqrt(K) rms(a) rms(b) for unscaled full-range codes, as
for the 8-bit tiles.
"""
import math

import numpy as np
import pytest

import oracle
import triton_ext_amd as tx
from dotcase import bits_to_f32, check_close, fp8_block_inputs, from_device, say, to_device
from test_dot_gpu import ATOL, RTOL

pytestmark = pytest.mark.gpu

OTYPE = {"e4m3": oracle.F8E4M3, "e5m2": oracle.F8E5M2}
TXTYPE = {"e4m3": tx.F8E4M3, "e5m2": tx.F8E5M2}


def codes(rng, shape, f):
    """Finite fp8 codes over the whole range (no NaN / Inf)."""
    c = rng.integers(0, 256, size=shape).astype(np.uint8)
    if f == "e5m2":
        return np.where((c & 0x7C) == 0x7C, c & 0x83, c).astype(np.uint8)
    return np.where((c & 0x7F) == 0x7F, c & 0xF0, c).astype(np.uint8)


def dec(q, f):
    return (oracle.e4m3_to_f32(q) if f == "e4m3"
            else oracle.f16_to_f32(q.astype(np.uint16) << 8)).astype(np.float64)


def tdt(f):
    import torch
    return {"e4m3": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}[f]


def up(x, m=16):
    return -(-x // m) * m


@pytest.mark.parametrize("fa,fb", [("e4m3", "e4m3"), ("e4m3", "e5m2"), ("e5m2", "e4m3"),
                                   ("e5m2", "e5m2")])
@pytest.mark.parametrize("M,N,K", [(16, 8192, 8192), (1, 4096, 4096), (64, 1024, 2048),
                                   (33, 1000, 3000), (7, 130, 129)])
def test_decode_f8_unscaled(gpu, fa, fb, M, N, K):
    import torch
    say(f"decode f8 {fa}x{fb} M={M} N={N} K={K}")
    rng = np.random.default_rng(M + N + K)
    a, b = codes(rng, (M, K), fa), codes(rng, (K, N), fb)
    p = tx.plan(tx.make_desc(M, N, K, TXTYPE[fa], tx.F32, b_type=TXTYPE[fb], lda=up(K),
                             ldb=up(N), ldc=up(N, 4)))
    assert p.kernel == tx.KERNEL_DECODE_F8
    c = tx.dot(to_device(a, gpu).view(tdt(fa)), to_device(b, gpu).view(tdt(fb)),
               out_dtype=torch.float32)
    torch.cuda.synchronize()
    got = from_device(c)
    ref = oracle.tiled_dot(a, b, a_type=OTYPE[fa], b_type=OTYPE[fb], c_type=oracle.F32,
                           block=(p.desc.block_m, p.desc.block_n, p.desc.block_k))
    rms = lambda q, f: float(np.sqrt(np.mean(dec(q, f) ** 2)))
    err = check_close(got, ref, atol=ATOL, rtol=RTOL, scale=math.sqrt(K) * rms(a, fa) * rms(b, fb),
                      what=f"decode f8 {fa}x{fb}")
    say(f"decode f8 {fa}x{fb} {M}x{N}x{K} split {p.split_k}: max|d|={err:.3g}")


@pytest.mark.parametrize("M,N,K,out", [(16, 7168, 7168, "bf16"), (1, 7168, 7168, "f32"),
                                       (64, 2048, 4096, "bf16"), (5, 1000, 2000, "f32"),
                                       (48, 384, 1000, "bf16"), (20, 256, 130, "f32")])
def test_decode_f8_block_scaled(gpu, M, N, K, out):
    """The block-scaled fp8 dot of decode shape (a K that fills no 128-block: the last
    block is partial)."""
    import torch
    say(f"decode f8 block-scaled M={M} N={N} K={K} out={out}")
    qa, qb, sa, sb = fp8_block_inputs(M, N, K, 7 + M)
    ct = oracle.F32 if out == "f32" else oracle.BF16
    p = tx.plan(tx.make_desc(M, N, K, tx.F8E4M3, tx.F32 if out == "f32" else tx.BF16,
                             scale_mode=tx.SCALE_BLOCK128, lda=up(K), ldb=up(N), ldc=up(N, 8)))
    assert p.kernel == tx.KERNEL_DECODE_F8
    c = tx.dot(to_device(qa, gpu), to_device(qb, gpu), scale_a=to_device(sa, gpu),
               scale_b=to_device(sb, gpu),
               out_dtype=torch.float32 if out == "f32" else torch.bfloat16)
    torch.cuda.synchronize()
    got = from_device(c)
    ref = oracle.tiled_dot(qa, qb, a_type=oracle.F8E4M3, c_type=ct, block=(128, 128, 128),
                           scale_mode=oracle.SCALE_BLOCK128, sa=sa, sb=sb)
    if out == "bf16":
        got, ref = bits_to_f32(got, "bf16"), bits_to_f32(ref, "bf16")
    err = check_close(got, ref, atol=ATOL, rtol=RTOL, scale=math.sqrt(K), what="decode f8 block")
    say(f"decode f8 block-scaled {M}x{N}x{K} split {p.split_k}: max|d|={err:.3g}")


def test_decode_f8_nan_padding_and_accumulate(gpu):
    """A and B in storage whose padding holds fp8 NaN codes (past K in A's rows, past N in
    B's, extra rows of B): the chunks that cross K or N are loaded whole, and the bytes
    past K must be zeroed (NaN * 0 = NaN).  With an fp32 acc: C = acc + A @ B."""
    import torch
    M, N, K = 9, 1001, 1003
    say(f"decode f8 NaN padding + acc M={M} N={N} K={K}")
    rng = np.random.default_rng(11)
    a, b = codes(rng, (M, K), "e4m3"), codes(rng, (K, N), "e4m3")
    A = np.full((M, K + 21), 0x7F, dtype=np.uint8)
    A[:, :K] = a
    B = np.full((K + 5, N + 7), 0xFF, dtype=np.uint8)
    B[:K, :N] = b
    acc = rng.standard_normal((M, N)).astype(np.float32)
    da = to_device(A, gpu).view(torch.float8_e4m3fn)
    db = to_device(B, gpu).view(torch.float8_e4m3fn)
    c = tx.dot(da[:, :K], db[:K, :N], out_dtype=torch.float32, acc=to_device(acc, gpu))
    torch.cuda.synchronize()
    got = from_device(c)
    assert np.isfinite(got).all()
    exact = dec(a, "e4m3") @ dec(b, "e4m3") + acc
    rms = lambda q: float(np.sqrt(np.mean(dec(q, "e4m3") ** 2)))
    check_close(got, exact.astype(np.float32), atol=ATOL, rtol=RTOL,
                scale=math.sqrt(K) * rms(a) * rms(b), what="decode f8 NaN padding")


def test_decode_f8_deterministic(gpu):
    """Split-K partials are summed in split order: the same bits on every launch."""
    import torch
    M, N, K = 16, 1024, 8192
    qa, qb, sa, sb = fp8_block_inputs(M, N, K, 3)
    p = tx.plan(tx.make_desc(M, N, K, tx.F8E4M3, tx.F32, scale_mode=tx.SCALE_BLOCK128))
    assert p.kernel == tx.KERNEL_DECODE_F8 and p.split_k == 16
    args = [to_device(x, gpu) for x in (qa, qb, sa, sb)]
    outs = []
    for _ in range(4):
        c = tx.dot(args[0], args[1], scale_a=args[2], scale_b=args[3], out_dtype=torch.float32)
        torch.cuda.synchronize()
        outs.append(from_device(c))
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32))
