"""Split-K on the 256x256 tiles: dots whose tile grid leaves most CUs idle (M of a
few hundred rows) cut K into ranges of whole steps, store 32-bit partial sums
and add them in range order in a second kernel that applies the dot's epilogue.

Against the oracle, with operands in padded storage whose padding holds NaN
(floating point) or random bytes (int8): int8 -> int32 and W8A8 bit-exact (the
int32 sums are exact in any order); fp16 / bf16 / fp8 within the north_star
tolerance (|d| <= 1e-3 s + 1e-2 |ref|) and, for fp32 C, within fp32 summation
error of the float64 product.  Ragged K puts the peeled K tail in the last
range.  The partials are added in range order, so repeated launches give the
same bits.
"""
import math

import numpy as np
import pytest

import oracle
import triton_ext_amd as tx
from dotcase import (bits_to_f32, check_close, fp8_block_inputs, from_device, k_norm, normal_bf16,
                     normal_f16, say, to_device, uniform_i8, uniform_scales)
from test_tails_gpu import dev_view, padded

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-3, 1e-2
NAN16 = {"bf16": 0x7FC0, "f16": 0x7E00}


def _plan(da, db, c, scale_mode=0, flags=0):
    return tx.plan_for(da, db, tx.tx_type(c), scale_mode, flags=flags, ldc=c.stride(0))


@pytest.mark.parametrize("M,N,K,kind,out,kmajor", [
    (256, 1024, 4096, "bf16", "bf16", False), (200, 1000, 4100, "bf16", "f32", False),
    (130, 777, 4001, "f16", "f16", False), (200, 1000, 4100, "f16", "f32", True),
    (300, 520, 8192, "bf16", "bf16", True), (100, 256, 2048, "bf16", "f32", False)])
def test_splitk_16bit(gpu, M, N, K, kind, out, kmajor):
    import torch
    say(f"split-K {kind}->{out} M={M} N={N} K={K} kmajor={kmajor}")
    gen = normal_bf16 if kind == "bf16" else normal_f16
    a, b = gen((M, K), k_norm(K), M + 1), gen((K, N), k_norm(K), N + 2)
    tdt = torch.bfloat16 if kind == "bf16" else torch.float16
    sa, _ = padded(a, NAN16[kind])
    da = dev_view(sa, (M, K), gpu, tdt)
    if kmajor:
        sbt, _ = padded(np.ascontiguousarray(b.T), NAN16[kind])
        db = dev_view(sbt, (N, K), gpu, tdt).t()
    else:
        sb, _ = padded(b, NAN16[kind])
        db = dev_view(sb, (K, N), gpu, tdt)
    odt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[out]
    c = tx.dot(da, db, out_dtype=odt)
    c2 = tx.dot(da, db, out_dtype=odt)
    torch.cuda.synchronize()
    p = _plan(da, db, c)
    assert p.kernel == tx.KERNEL_GEMM_16BIT and p.split_k > 1 and p.grid_y == p.split_k
    assert (p.desc.block_m, p.desc.block_n) == (256, 256)
    assert bool(p.desc.flags & tx.FLAG_B_KMAJOR) == kmajor
    at = oracle.BF16 if kind == "bf16" else oracle.F16
    ct = {"f32": oracle.F32, "bf16": oracle.BF16, "f16": oracle.F16}[out]
    ref = oracle.tiled_dot(a, b, a_type=at, c_type=ct, block=(256, 256, 64))
    got = from_device(c)
    assert np.array_equal(got.view(np.uint8), from_device(c2).view(np.uint8))
    err = check_close(bits_to_f32(got, out), bits_to_f32(ref, out), atol=ATOL, rtol=RTOL,
                      what=f"split-K {kind} {M}x{N}x{K}")
    if out == "f32":
        f = oracle.bf16_to_f32 if kind == "bf16" else oracle.f16_to_f32
        exact = f(a).astype(np.float64) @ f(b).astype(np.float64)
        assert np.abs(got - exact).max() < 1e-5
    say(f"split {p.split_k}: max|d|={err:.3g}")


def test_splitk_accumulate(gpu):
    """tl.dot(a, b, acc) with split-K: C = acc + A @ B, the reduction adds acc once."""
    import torch
    M, N, K = 200, 1000, 4096
    say(f"split-K acc M={M} N={N} K={K}")
    a, b = normal_bf16((M, K), k_norm(K), 5), normal_bf16((K, N), k_norm(K), 6)
    acc = np.random.default_rng(7).standard_normal((M, N)).astype(np.float32)
    da, db = to_device(a, gpu).view(torch.bfloat16), to_device(b, gpu).view(torch.bfloat16)
    c = tx.dot(da, db, acc=to_device(acc, gpu))
    torch.cuda.synchronize()
    p = tx.plan_for(da, db, tx.F32, flags=tx.FLAG_ACCUMULATE, ldc=c.stride(0))
    assert p.split_k > 1
    exact = oracle.bf16_to_f32(a).astype(np.float64) @ oracle.bf16_to_f32(b).astype(np.float64)
    assert np.abs(from_device(c) - (exact + acc)).max() < 1e-5


@pytest.mark.parametrize("M,N,K,scaled,kmajor", [
    (600, 1000, 4100, False, False), (700, 520, 8192, True, False),
    (600, 1000, 4100, True, True), (1024, 1024, 4096, False, True)])
def test_splitk_int8(gpu, M, N, K, scaled, kmajor):
    """int8 -> int32 and W8A8 past the row decode kernel's M = 512, on the 256x256x128 tile
    with split-K: int32 partials, bit-exact against the oracle (junk in the padding)."""
    import torch
    say(f"split-K int8 M={M} N={N} K={K} scaled={scaled} kmajor={kmajor}")
    a, b = uniform_i8((M, K), 11), uniform_i8((K, N), 12)
    junk = np.random.default_rng(13)
    pa, _ = padded(a, 0)
    pa[:, K:] = junk.integers(-128, 128, size=pa[:, K:].shape)
    da = dev_view(pa, (M, K), gpu)
    src = np.ascontiguousarray(b.T) if kmajor else b
    pb, _ = padded(src, 0)
    pb[:, src.shape[1]:] = junk.integers(-128, 128, size=pb[:, src.shape[1]:].shape)
    pb[src.shape[0]:, :] = junk.integers(-128, 128, size=pb[src.shape[0]:, :].shape)
    db = dev_view(pb, src.shape, gpu)
    db = db.t() if kmajor else db
    if scaled:
        sa, sb = uniform_scales(M, 14), uniform_scales(N, 15)
        c = tx.dot(da, db, scale_a=to_device(sa, gpu), scale_b=to_device(sb, gpu),
                   out_dtype=torch.bfloat16)
        ref = oracle.tiled_dot(a, b, a_type=oracle.I8, c_type=oracle.BF16, block=(64, 64, 64),
                               scale_mode=oracle.SCALE_ROWCOL, sa=sa, sb=sb)
    else:
        c = tx.dot(da, db, out_dtype=torch.int32)
        ref = oracle.tiled_dot(a, b, a_type=oracle.I8, c_type=oracle.I32, block=(64, 64, 64))
    torch.cuda.synchronize()
    p = _plan(da, db, c, tx.SCALE_ROWCOL if scaled else 0)
    assert p.kernel == tx.KERNEL_GEMM_I8 and p.split_k > 1
    got = from_device(c)
    assert np.array_equal(got, ref), f"{np.count_nonzero(got != ref)} mismatches"


@pytest.mark.parametrize("M,N,K,out,kmajor", [
    (256, 7168, 7168, "bf16", False), (200, 1000, 4096, "f32", False),
    (200, 1000, 4096, "bf16", True), (130, 300, 4000, "bf16", False)])
def test_splitk_fp8_block_scaled(gpu, M, N, K, out, kmajor):
    """The block-scaled fp8 dot (config 4's form) at M of a few hundred rows: the tile's
    scaled fp32 partials over whole 128-K blocks, NaN codes in the padding."""
    import torch
    say(f"split-K fp8 block M={M} N={N} K={K} out={out} kmajor={kmajor}")
    qa, qb, sa, sb = fp8_block_inputs(M, N, K, 21)
    pa, _ = padded(qa, 0x7F)
    da = dev_view(pa, (M, K), gpu, torch.float8_e4m3fn)
    src = np.ascontiguousarray(qb.T) if kmajor else qb
    pb, _ = padded(src, 0x7F)
    db = dev_view(pb, src.shape, gpu, torch.float8_e4m3fn)
    db = db.t() if kmajor else db
    odt = torch.bfloat16 if out == "bf16" else torch.float32
    c = tx.dot(da, db, scale_a=to_device(sa, gpu), scale_b=to_device(sb, gpu), out_dtype=odt)
    torch.cuda.synchronize()
    p = _plan(da, db, c, tx.SCALE_BLOCK128)
    assert p.kernel == tx.KERNEL_GEMM_F8 and p.split_k > 1
    ct = oracle.BF16 if out == "bf16" else oracle.F32
    ref = oracle.tiled_dot(qa, qb, a_type=oracle.F8E4M3, c_type=ct, block=(128, 128, 128),
                           scale_mode=oracle.SCALE_BLOCK128, sa=sa, sb=sb)
    got = from_device(c)
    if out == "bf16":
        got, ref = bits_to_f32(got, "bf16"), bits_to_f32(ref, "bf16")
    check_close(got, ref, atol=ATOL, rtol=RTOL, scale=math.sqrt(K), what="split-K fp8 block")


@pytest.mark.parametrize("fa,fb", [("e4m3", "e4m3"), ("e5m2", "e4m3")])
def test_splitk_fp8_unscaled(gpu, fa, fb):
    import torch
    M, N, K = 100, 777, 4096
    say(f"split-K fp8 {fa}x{fb} M={M} N={N} K={K}")
    rng = np.random.default_rng(31)

    def codes(shape, f):
        c = rng.integers(0, 256, size=shape).astype(np.uint8)
        if f == "e5m2":
            return np.where((c & 0x7C) == 0x7C, c & 0x83, c).astype(np.uint8)
        return np.where((c & 0x7F) == 0x7F, c & 0xF0, c).astype(np.uint8)
    a, b = codes((M, K), fa), codes((K, N), fb)
    tdt = {"e4m3": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}
    otype = {"e4m3": oracle.F8E4M3, "e5m2": oracle.F8E5M2}
    da = to_device(a, gpu).view(tdt[fa])
    pb, _ = padded(b, 0x7F)
    db = dev_view(pb, (K, N), gpu, tdt[fb])
    c = tx.dot(da, db, out_dtype=torch.float32)
    torch.cuda.synchronize()
    p = _plan(da, db, c)
    assert p.kernel == tx.KERNEL_GEMM_F8 and p.split_k > 1
    ref = oracle.tiled_dot(a, b, a_type=otype[fa], b_type=otype[fb], c_type=oracle.F32,
                           block=(256, 256, 128))
    dec = lambda q, f: (oracle.e4m3_to_f32(q) if f == "e4m3"
                        else oracle.f16_to_f32(q.astype(np.uint16) << 8)).astype(np.float64)
    rms = lambda q, f: float(np.sqrt(np.mean(dec(q, f) ** 2)))
    check_close(from_device(c), ref, atol=ATOL, rtol=RTOL,
                scale=math.sqrt(K) * rms(a, fa) * rms(b, fb), what="split-K fp8")
