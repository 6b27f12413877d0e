"""GPU parity for K and N that do not fill whole 16-byte chunks.

Triton's masked tl.load (T:runtime/interpreter.py:449-455) zero-fills every
element past K and drops every column past N, whatever K and N are; the
reference kernel's K loop has the same shape (R:pass/LoopSplit/LoopSplit.cpp
:156-174 peels the masked step).  Here every operand lives in padded storage
whose padding holds NaN (floating point) or random bytes (int8), with extra
rows past M (A) and past K (B) holding the same: an element past an edge
that reached the MFMA would turn a result into NaN or change an integer sum.

Bars: int8 and W8A8 bit-exact; fp16/bf16/fp8 within the north_star tolerance
(|d| <= 1e-3 s + 1e-2 |ref|, s as in test_dot_gpu.py).
"""
import math

import numpy as np
import pytest

import oracle
import triton_ext_amd as tx
from dotcase import (bits_to_f32, check_close, fp8_block_inputs, from_device, k_norm, normal_bf16,
                     normal_f16, say, to_device, uniform_i8, uniform_scales)

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-3, 1e-2
NAN16 = {"bf16": 0x7FC0, "f16": 0x7E00}


def padded(x, fill, extra_rows=3, quantum=16):
    """x [R, C] (numpy) inside storage [R + extra_rows, C'], the rest `fill`.
    C' is C rounded up to whole 16-byte chunks, plus one chunk when C fills
    its last chunk exactly, so every row has padding.  Returns (storage, C')."""
    elt = x.dtype.itemsize
    per = quantum // elt
    ld = -(-x.shape[1] // per) * per
    if ld == x.shape[1]:
        ld += per  # padding on every row, also when C is chunk-aligned
    st = np.full((x.shape[0] + extra_rows, ld), fill, dtype=x.dtype)
    st[:x.shape[0], :x.shape[1]] = x
    return st, ld


def dev_view(st, shape, gpu, tdtype=None):
    t = to_device(st, gpu)
    if tdtype is not None:
        t = t.view(tdtype)
    return t[:shape[0], :shape[1]]


def run16(gpu, M, N, K, kind, out_kind, block=(0, 0, 0), kmajor=False, seed=0):
    import torch
    say(f"tails {kind}->{out_kind} M={M} N={N} K={K} block={block} kmajor={kmajor}")
    gen = normal_bf16 if kind == "bf16" else normal_f16
    a = gen((M, K), k_norm(K), 51 + seed)
    b = gen((K, N), k_norm(K), 52 + seed)
    tdt = torch.bfloat16 if kind == "bf16" else torch.float16
    sa, _ = padded(a, NAN16[kind])
    da = dev_view(sa, (M, K), gpu, tdt)
    if kmajor:  # B stored [N][K]: its rows past N and columns past K hold NaN
        sbt, _ = padded(np.ascontiguousarray(b.T), NAN16[kind])
        db = dev_view(sbt, (N, K), gpu, tdt).t()
    else:
        sb, _ = padded(b, NAN16[kind])
        db = dev_view(sb, (K, N), gpu, tdt)
    out_dt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[out_kind]
    c = tx.dot(da, db, out_dtype=out_dt, block=block)
    torch.cuda.synchronize()
    p = tx.plan_for(da, db, tx.tx_type(c), block=block, ldc=c.stride(0))
    blk = (p.desc.block_m, p.desc.block_n, p.desc.block_k)
    at = oracle.BF16 if kind == "bf16" else oracle.F16
    ct = {"f32": oracle.F32, "bf16": oracle.BF16, "f16": oracle.F16}[out_kind]
    ref = oracle.tiled_dot(a, b, a_type=at, c_type=ct, block=blk)
    got = from_device(c)
    okind = "f32" if out_kind == "f32" else out_kind
    err = check_close(bits_to_f32(got, okind), bits_to_f32(ref, okind), atol=ATOL, rtol=RTOL,
                      what=f"{kind} {M}x{N}x{K}")
    say(f"max|d|={err:.3g} tile={blk}")
    return p


@pytest.mark.parametrize("M,N,K", [(4001, 4001, 4001), (4096, 4096, 4001)])
def test_bf16_ragged_headline_shapes(gpu, M, N, K):
    """bf16 4001^3 and 4096 x 4096 x 4001 on the 256x256 tile: K tail of 33 (4001 = 62 * 64
    + 33) with a chunk crossing K, and (4001^3) edge tiles whose last chunk crosses N."""
    p = run16(gpu, M, N, K, "bf16", "bf16")
    assert (p.desc.block_m, p.desc.block_n) == (256, 256) and p.k_tail == K % 64


@pytest.mark.parametrize("M,N,K,kind,out,block", [
    (300, 261, 203, "bf16", "f32", (0, 0, 0)),
    (257, 259, 131, "f16", "f16", (0, 0, 0)),
    (33, 17, 9, "bf16", "bf16", (0, 0, 0)),
    (300, 261, 203, "bf16", "f32", (128, 128, 64)),
    (129, 67, 45, "f16", "f32", (64, 64, 32)),
    (70, 35, 1, "f16", "f16", (64, 64, 32)),
])
def test_16bit_ragged(gpu, M, N, K, kind, out, block):
    run16(gpu, M, N, K, kind, out, block)


@pytest.mark.parametrize("M,N,K,block", [(300, 261, 203, (0, 0, 0)), (64, 50, 70, (256, 256, 64)),
                                         (64, 50, 70, (0, 0, 0)), (90, 50, 70, (0, 0, 0))])
def test_16bit_ragged_kmajor_b(gpu, M, N, K, block):
    """K-major B (q @ k.T): B's chunk that crosses K is zeroed in registers too, on the
    256 tile and (M <= 96, the planner's choice) the decode kernel."""
    p = run16(gpu, M, N, K, "bf16", "f32", block=block, kmajor=True)
    assert p.kernel == (tx.KERNEL_DECODE_16BIT if M <= 96 and block == (0, 0, 0)
                        else tx.KERNEL_GEMM_16BIT)


@pytest.mark.parametrize("M,N,K,block", [(300, 261, 203, (256, 256, 128)),
                                         (300, 261, 203, (128, 128, 128)),
                                         (17, 1001, 999, (0, 0, 0))])
def test_int8_ragged(gpu, M, N, K, block):
    """int8 -> int32, bit-exact; the padding holds random bytes."""
    import torch
    say(f"tails int8 M={M} N={N} K={K} block={block}")
    a = uniform_i8((M, K), 61)
    b = uniform_i8((K, N), 62)
    junk = np.random.default_rng(63)
    sa, _ = padded(a, 0)
    sa[:, K:] = junk.integers(-128, 128, size=sa[:, K:].shape)
    sa[M:, :] = junk.integers(-128, 128, size=sa[M:, :].shape)
    sb, _ = padded(b, 0)
    sb[:, N:] = junk.integers(-128, 128, size=sb[:, N:].shape)
    sb[K:, :] = junk.integers(-128, 128, size=sb[K:, :].shape)
    c = tx.dot(dev_view(sa, (M, K), gpu), dev_view(sb, (K, N), gpu), out_dtype=torch.int32,
               block=block)
    torch.cuda.synchronize()
    ref = oracle.tiled_dot(a, b, a_type=oracle.I8, c_type=oracle.I32, block=(64, 64, 64))
    assert np.array_equal(from_device(c), ref)


@pytest.mark.parametrize("N", [49, 50, 51, 53, 55])
@pytest.mark.parametrize("out", ["f32", "bf16"])
@pytest.mark.parametrize("kmajor", [False, True])
def test_16bit_every_element_of_the_chunk_crossing_n(gpu, N, out, kmajor):
    """The 256 tile's edge epilogue stores the chunk that crosses N element by element:
    N mod 4 (fp32 C) and N mod 8 (bf16 C) take every value the chunk can leave.  (M = 64
    would take the decode kernel: the tile is named.)"""
    p = run16(gpu, 64, N, 70, "bf16", out, block=(256, 256, 64), kmajor=kmajor)
    assert p.kernel == tx.KERNEL_GEMM_16BIT


@pytest.mark.parametrize("N", [49, 50, 51])
def test_8bit_every_element_of_the_quad_crossing_n(gpu, N):
    """The 8-bit tile's edge epilogue: int8 -> int32 with N mod 4 = 1, 2, 3, bit-exact."""
    import torch
    M, K = 40, 200
    say(f"tails int8 quad crossing N M={M} N={N} K={K}")
    a, b = uniform_i8((M, K), 64), uniform_i8((K, N), 65)
    sa, _ = padded(a, 0)
    sb, _ = padded(b, 0)
    c = tx.dot(dev_view(sa, (M, K), gpu), dev_view(sb, (K, N), gpu), out_dtype=torch.int32,
               block=(256, 256, 128))
    torch.cuda.synchronize()
    ref = oracle.tiled_dot(a, b, a_type=oracle.I8, c_type=oracle.I32, block=(64, 64, 64))
    assert np.array_equal(from_device(c), ref)


def _fp8_codes(shape, seed):
    c = np.random.default_rng(seed).integers(0, 256, size=shape).astype(np.uint8)
    return np.where((c & 0x7F) == 0x7F, c & 0xF0, c).astype(np.uint8)  # no NaN codes


@pytest.mark.parametrize("M,N,K,block", [(300, 263, 391, (256, 256, 128)),
                                         (300, 263, 391, (256, 224, 128)),
                                         (300, 263, 391, (128, 128, 128))])
def test_fp8_ragged_unscaled(gpu, M, N, K, block):
    """e4m3 -> fp32 with NaN codes (0x7F) in A's and B's padding: A's bytes past K must be
    zeroed before the MFMA (NaN times B's zero rows is still NaN)."""
    import torch
    say(f"tails fp8 M={M} N={N} K={K} block={block}")
    a, b = _fp8_codes((M, K), 71), _fp8_codes((K, N), 72)
    sa, _ = padded(a, 0x7F)
    sb, _ = padded(b, 0x7F)
    c = tx.dot(dev_view(sa, (M, K), gpu, torch.float8_e4m3fn),
               dev_view(sb, (K, N), gpu, torch.float8_e4m3fn), out_dtype=torch.float32,
               block=block)
    torch.cuda.synchronize()
    ref = oracle.tiled_dot(a, b, a_type=oracle.F8E4M3, c_type=oracle.F32, block=(128, 128, 128))
    fa, fb = oracle.e4m3_to_f32(a).astype(np.float64), oracle.e4m3_to_f32(b).astype(np.float64)
    s = math.sqrt(K) * math.sqrt((fa ** 2).mean()) * math.sqrt((fb ** 2).mean())
    check_close(from_device(c), ref, atol=ATOL, rtol=RTOL, scale=s, what="fp8 ragged")


@pytest.mark.parametrize("M,N,K,block", [(2048, 7167, 7168, (0, 0, 0)),
                                         (300, 263, 391, (256, 256, 128)),
                                         (300, 263, 391, (256, 224, 128)),
                                         (300, 263, 391, (128, 128, 128))])
def test_fp8_block_scaled_ragged(gpu, M, N, K, block):
    """Config 4's dot with N = 7167 (a last chunk crossing N, a partial 128-column scale
    block), and smaller ragged shapes on each 8-bit tile."""
    import torch
    say(f"tails fp8 block-scaled M={M} N={N} K={K} block={block}")
    qa, qb, sa, sb = fp8_block_inputs(M, N, K, 73)
    pa, _ = padded(qa, 0x7F)
    pb, _ = padded(qb, 0x7F)
    c = tx.dot(dev_view(pa, (M, K), gpu, torch.float8_e4m3fn),
               dev_view(pb, (K, N), gpu, torch.float8_e4m3fn),
               scale_a=to_device(sa, gpu), scale_b=to_device(sb, gpu), out_dtype=torch.bfloat16,
               block=block)
    torch.cuda.synchronize()
    ref = oracle.tiled_dot(qa, qb, a_type=oracle.F8E4M3, c_type=oracle.BF16, block=(128, 128, 128),
                           scale_mode=oracle.SCALE_BLOCK128, sa=sa, sb=sb)
    check_close(bits_to_f32(from_device(c), "bf16"), bits_to_f32(ref, "bf16"), atol=ATOL,
                rtol=RTOL, scale=math.sqrt(K), what="fp8 block ragged")


@pytest.mark.parametrize("M,N,K", [(16, 8192, 8191), (16, 8191, 8192), (5, 1001, 999),
                                   (100, 3001, 2049), (1, 17, 15)])
def test_w8a8_ragged(gpu, M, N, K):
    """W8A8 decode with K or N not a multiple of 16 (config 3's N = K = 8192 less one):
    bit-exact."""
    import torch
    say(f"tails W8A8 M={M} N={N} K={K}")
    a = uniform_i8((M, K), 81)
    b = uniform_i8((K, N), 82)
    sa_, sb_ = uniform_scales(M, 83), uniform_scales(N, 84)
    junk = np.random.default_rng(85)
    pa, _ = padded(a, 0)
    pa[:, K:] = junk.integers(-128, 128, size=pa[:, K:].shape)
    pb, _ = padded(b, 0)
    pb[:, N:] = junk.integers(-128, 128, size=pb[:, N:].shape)
    pb[K:, :] = junk.integers(-128, 128, size=pb[K:, :].shape)
    da, db = dev_view(pa, (M, K), gpu), dev_view(pb, (K, N), gpu)
    c = tx.new_output(M, N, torch.bfloat16, gpu)
    p = tx.plan(tx.make_desc(M, N, K, tx.I8, tx.BF16, scale_mode=tx.SCALE_ROWCOL,
                             lda=da.stride(0), ldb=db.stride(0), ldc=c.stride(0)))
    assert p.kernel == tx.KERNEL_DECODE_I8
    tx.dot(da, db, scale_a=to_device(sa_, gpu), scale_b=to_device(sb_, gpu), out=c)
    torch.cuda.synchronize()
    ref = oracle.tiled_dot(a, b, a_type=oracle.I8, c_type=oracle.BF16, block=(64, 256, 128),
                           scale_mode=oracle.SCALE_ROWCOL, sa=sa_, sb=sb_)
    got = from_device(c)
    assert np.array_equal(got, ref), f"{np.count_nonzero(got != ref)} mismatches"


def test_mx_ragged_n(gpu):
    """tl.dot_scaled (e8m0 per 32) with N not a multiple of 16: the last B chunk crosses N."""
    import torch
    M, N, K = 200, 250, 256
    say(f"tails mx M={M} N={N} K={K}")
    a, b = _fp8_codes((M, K), 91), _fp8_codes((K, N), 92)
    rng = np.random.default_rng(93)
    sa = rng.integers(120, 134, size=(M, K // 32)).astype(np.uint8)
    sbs = rng.integers(120, 134, size=(N, K // 32)).astype(np.uint8)
    pb, _ = padded(b, 0x7F)
    c = tx.dot_scaled(to_device(a, gpu), to_device(sa, gpu), "e4m3",
                      dev_view(pb, (K, N), gpu), to_device(sbs, gpu), "e4m3")
    torch.cuda.synchronize()
    ref = oracle.dot_scaled(a, sa, oracle.F8E4M3, b, sbs, oracle.F8E4M3, K=K)
    fa = oracle.e4m3_to_f32(a).astype(np.float64) * np.exp2(np.repeat(sa, 32, 1).astype(np.float64) - 127)
    fb = oracle.e4m3_to_f32(b).astype(np.float64) * np.exp2(np.repeat(sbs, 32, 1).T.astype(np.float64) - 127)
    s = math.sqrt(K) * math.sqrt((fa ** 2).mean()) * math.sqrt((fb ** 2).mean())
    check_close(from_device(c), ref, atol=ATOL, rtol=RTOL, scale=s, what="mx ragged N")


def test_accumulate_ragged_n(gpu):
    """acc + A @ B with N = 261: the quads that cross N are added element by element."""
    import torch
    M, N, K = 300, 261, 203
    say(f"tails accumulate M={M} N={N} K={K}")
    a = normal_bf16((M, K), k_norm(K), 101)
    b = normal_bf16((K, N), k_norm(K), 102)
    acc = np.random.default_rng(103).standard_normal((M, N)).astype(np.float32)
    da = to_device(a, gpu).view(torch.bfloat16)
    db = to_device(b, gpu).view(torch.bfloat16)
    plain = tx.dot(da, db, out_dtype=torch.float32)
    got = tx.dot(da, db, acc=to_device(acc, gpu))
    torch.cuda.synchronize()
    # the result is exactly the plain result plus acc in one fp32 addition
    want = (from_device(plain).astype(np.float32) + acc).astype(np.float32)
    assert np.array_equal(from_device(got), want)


def test_contiguous_unaligned_operands(gpu):
    """dot() on contiguous [M, K] / [K, N] tensors with rows 8002 bytes apart: the binding
    copies them into 16-byte-aligned rows; the result matches the oracle."""
    import torch
    M = N = K = 1001
    say(f"tails contiguous unaligned {M}x{N}x{K}")
    a = normal_bf16((M, K), k_norm(K), 111)
    b = normal_bf16((K, N), k_norm(K), 112)
    da = to_device(a, gpu).view(torch.bfloat16)
    db = to_device(b, gpu).view(torch.bfloat16)
    assert da.stride(0) * 2 % 16 != 0
    c = tx.dot(da, db, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert c.shape == (M, N) and (c.stride(0) * 2) % 16 == 0
    p = tx.plan(tx.make_desc(M, N, K, tx.BF16, tx.BF16, lda=1008, ldb=1008, ldc=1008))
    ref = oracle.tiled_dot(a, b, a_type=oracle.BF16, c_type=oracle.BF16,
                           block=(p.desc.block_m, p.desc.block_n, p.desc.block_k))
    check_close(bits_to_f32(from_device(c), "bf16"), bits_to_f32(ref, "bf16"), atol=ATOL,
                rtol=RTOL, what="contiguous unaligned")


@pytest.mark.parametrize("M,N,block", [(5, 220, (0, 0, 0)), (64, 3, (0, 0, 0)),
                                       (5, 220, (256, 256, 64))])
def test_16bit_k1_kmajor_b(gpu, M, N, block):
    """K = 1 with B a transposed view (q @ k.T with one head dim): the single row of B has
    elements ldk apart, which is the K-major layout; the stride of a size-1 dimension says
    nothing about the layout.  The decode kernel (the planner's choice) and the 256 tile."""
    p = run16(gpu, M, N, 1, "bf16", "f32", block=block, kmajor=True)
    assert p.desc.flags & tx.FLAG_B_KMAJOR


@pytest.mark.parametrize("out", ["i32", "bf16"])
def test_single_column_b_from_a_transposed_row(gpu, out):
    """N = 1 with B = x.t() for x [1, K]: a single column whose column stride is K.  Its
    elements are adjacent, so an int32 or bf16 dot runs it K-major (after a copy into
    16-byte rows here, K = 300 not being a multiple of 16 bytes)."""
    import torch
    M, K = 40, 300
    say(f"tails single-column B {out}")
    if out == "i32":
        a, x = uniform_i8((M, K), 71), uniform_i8((1, K), 72)
        c = tx.dot(to_device(a, gpu), to_device(x, gpu).t(), out_dtype=torch.int32)
        torch.cuda.synchronize()
        ref = oracle.tiled_dot(a, np.ascontiguousarray(x.T), a_type=oracle.I8, c_type=oracle.I32,
                               block=(64, 64, 64))
        assert np.array_equal(from_device(c), ref)
    else:
        a, x = normal_bf16((M, K), k_norm(K), 73), normal_bf16((1, K), k_norm(K), 74)
        c = tx.dot(to_device(a, gpu).view(torch.bfloat16), to_device(x, gpu).view(torch.bfloat16).t(),
                   out_dtype=torch.bfloat16)
        torch.cuda.synchronize()
        ref = oracle.tiled_dot(a, np.ascontiguousarray(x.T), a_type=oracle.BF16, c_type=oracle.BF16,
                               block=(64, 64, 32))
        check_close(bits_to_f32(from_device(c), "bf16"), bits_to_f32(ref, "bf16"), atol=ATOL,
                    rtol=RTOL, what="single-column B")


def _codes8(rng, shape, f):
    """Finite fp8 codes over the whole range (no NaN / Inf)."""
    c = rng.integers(0, 256, size=shape).astype(np.uint8)
    if f == "e5m2":
        return np.where((c & 0x7C) == 0x7C, c & 0x83, c).astype(np.uint8)
    return np.where((c & 0x7F) == 0x7F, c & 0xF0, c).astype(np.uint8)


def _kmajor_b(b, fill, gpu, tdtype=None, junk=None):
    """B [K, N] as a transposed view of [N][K'] storage: columns past K and rows past N hold
    `fill`, or random bytes from `junk`."""
    N, K = b.shape[1], b.shape[0]
    st, _ = padded(np.ascontiguousarray(b.T), fill)
    if junk is not None:
        st[:, K:] = junk.integers(-128, 128, size=st[:, K:].shape)
        st[N:, :] = junk.integers(-128, 128, size=st[N:, :].shape)
    return dev_view(st, (N, K), gpu, tdtype).t()


def _kmajor_kernel(M, kernel, block, i8):
    """The kernel a K-major 8-bit plan takes: with the planner's choice the 8-bit decode
    kernel at M <= 64 (int8: M <= 48) and for int8 the row decode kernel beyond, to
    M = 256; else the 256x256x128 tile (`kernel`)."""
    if block != (0, 0, 0):
        return kernel
    if M <= (48 if i8 else 64):
        return tx.KERNEL_DECODE_F8
    return tx.KERNEL_DECODE_I8 if i8 and M <= 256 else kernel


def _assert_kmajor_plan(da, db, c, kernel, block=(0, 0, 0), scale_mode=0):
    """The plan is K-major, on the kernel _kmajor_kernel names; returns it."""
    p = tx.plan_for(da, db, tx.tx_type(c), scale_mode, block=block, ldc=c.stride(0))
    assert p.desc.flags & tx.FLAG_B_KMAJOR
    want = _kmajor_kernel(da.shape[0], kernel, block, da.element_size() == 1 and
                          kernel == tx.KERNEL_GEMM_I8)
    assert p.kernel == want
    if want == kernel:
        assert (p.desc.block_m, p.desc.block_n, p.desc.block_k) == (256, 256, 128)
    return p


@pytest.mark.parametrize("M,N,K,block", [
    (300, 263, 391, (0, 0, 0)), (512, 512, 1024, (0, 0, 0)),
    (40, 50, 200, (0, 0, 0)), (17, 1001, 999, (0, 0, 0)), (5, 220, 1, (0, 0, 0)),
    (64, 3, 129, (0, 0, 0)), (16, 4096, 4096, (0, 0, 0)), (33, 300, 4001, (0, 0, 0)),
    (40, 50, 200, (256, 256, 128)), (17, 1001, 999, (256, 256, 128)),
    (5, 220, 1, (256, 256, 128)), (64, 3, 129, (256, 256, 128)),
    (300, 263, 391, (256, 256, 128)), (129, 8192, 4096, (0, 0, 0))])
def test_int8_ragged_kmajor_b(gpu, M, N, K, block):
    """int8 -> int32 with B a transposed view (q @ k.T): B's padding columns past K and rows
    past N hold random bytes, as do A's.  The chunk that crosses K is loaded whole on both
    sides, so both are zeroed past K (junk times junk is not zero).  Bit-exact, on the
    256x256x128 tile and, with the planner's choice, the 8-bit decode kernel (M <= 48) and
    the row decode kernel (48 < M <= 256)."""
    import torch
    say(f"tails int8 K-major B M={M} N={N} K={K} block={block}")
    a, b = uniform_i8((M, K), 81), uniform_i8((K, N), 82)
    junk = np.random.default_rng(83)
    sa, _ = padded(a, 0)
    sa[:, K:] = junk.integers(-128, 128, size=sa[:, K:].shape)
    sa[M:, :] = junk.integers(-128, 128, size=sa[M:, :].shape)
    da = dev_view(sa, (M, K), gpu)
    db = _kmajor_b(b, 0, gpu, junk=junk)
    c = tx.dot(da, db, out_dtype=torch.int32, block=block)
    torch.cuda.synchronize()
    _assert_kmajor_plan(da, db, c, tx.KERNEL_GEMM_I8, block)
    ref = oracle.tiled_dot(a, b, a_type=oracle.I8, c_type=oracle.I32, block=(64, 64, 64))
    assert np.array_equal(from_device(c), ref)


@pytest.mark.parametrize("fa,fb", [("e4m3", "e4m3"), ("e4m3", "e5m2"), ("e5m2", "e4m3"),
                                   ("e5m2", "e5m2")])
@pytest.mark.parametrize("M,N,K,block", [(300, 263, 391, (0, 0, 0)), (130, 77, 1, (0, 0, 0)),
                                         (16, 1024, 256, (256, 256, 128)),
                                         (16, 1024, 256, (0, 0, 0)), (33, 777, 1001, (0, 0, 0)),
                                         (1, 4096, 4096, (0, 0, 0))])
def test_fp8_ragged_kmajor_b(gpu, fa, fb, M, N, K, block):
    """Unscaled fp8 -> fp32 with B a transposed view, NaN codes (0x7F, NaN in e4m3 and
    e5m2) in both operands' padding; e4m3 / e5m2 in every mix.  Against the oracle; on the
    256 tile also bit for bit against the same dot with B row-major (the K-major fragment
    holds the same K indices in the same bytes).  M <= 64 with the planner's choice runs
    the 8-bit decode kernel."""
    import torch
    say(f"tails fp8 K-major B {fa}x{fb} M={M} N={N} K={K} block={block}")
    rng = np.random.default_rng(M + N + K)
    a, b = _codes8(rng, (M, K), fa), _codes8(rng, (K, N), fb)
    tdt = {"e4m3": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}
    otype = {"e4m3": oracle.F8E4M3, "e5m2": oracle.F8E5M2}
    sa, _ = padded(a, 0x7F)
    da = dev_view(sa, (M, K), gpu, tdt[fa])
    db = _kmajor_b(b, 0x7F, gpu, tdt[fb])
    c = tx.dot(da, db, out_dtype=torch.float32, block=block)
    sb, _ = padded(b, 0x7F)
    c_row = tx.dot(da, dev_view(sb, (K, N), gpu, tdt[fb]), out_dtype=torch.float32,
                   block=(256, 256, 128))
    torch.cuda.synchronize()
    p = _assert_kmajor_plan(da, db, c, tx.KERNEL_GEMM_F8, block)
    got = from_device(c)
    ref = oracle.tiled_dot(a, b, a_type=otype[fa], b_type=otype[fb], c_type=oracle.F32,
                           block=(256, 256, 128))
    dec = lambda q, f: (oracle.e4m3_to_f32(q) if f == "e4m3"
                        else oracle.f16_to_f32(q.astype(np.uint16) << 8)).astype(np.float64)
    rms = lambda q, f: float(np.sqrt(np.mean(dec(q, f) ** 2)))
    check_close(got, ref, atol=ATOL, rtol=RTOL, scale=math.sqrt(K) * rms(a, fa) * rms(b, fb),
                what=f"fp8 K-major {fa}x{fb}")
    if p.kernel == tx.KERNEL_GEMM_F8:
        assert np.array_equal(got.view(np.uint32), from_device(c_row).view(np.uint32))


@pytest.mark.parametrize("kind", ["i8", "e4m3"])
def test_8bit_kmajor_b_full_size(gpu, kind):
    """4096 x 4096 x 4096 (the int8 headline shape) with B = k.t(): bit for bit the dot
    with B row-major, whose parity the oracle pins at the smaller sizes."""
    import torch
    M = N = K = 4096
    say(f"tails 8-bit K-major B full size {kind}")
    g = torch.Generator(device=gpu)
    g.manual_seed(91)
    if kind == "i8":
        a = torch.randint(-128, 128, (M, K), generator=g, device=gpu, dtype=torch.int8)
        k = torch.randint(-128, 128, (N, K), generator=g, device=gpu, dtype=torch.int8)
        odt, kern = torch.int32, tx.KERNEL_GEMM_I8
    else:
        a = torch.randn((M, K), generator=g, device=gpu).to(torch.float8_e4m3fn)
        k = torch.randn((N, K), generator=g, device=gpu).to(torch.float8_e4m3fn)
        odt, kern = torch.float32, tx.KERNEL_GEMM_F8
    c = tx.dot(a, k.t(), out_dtype=odt)
    c_row = tx.dot(a, k.t().contiguous(), out_dtype=odt, block=(256, 256, 128))
    torch.cuda.synchronize()
    _assert_kmajor_plan(a, k.t(), c, kern)
    assert torch.equal(c.view(torch.int32), c_row.view(torch.int32))


@pytest.mark.parametrize("kind,M", [("i8", 16), ("e4m3", 16), ("i8", 100)])
def test_8bit_kmajor_decode_accumulate(gpu, kind, M):
    """tl.dot(a, k.T, acc) at decode shape on the 8-bit decode kernel (M = 16) and the row
    decode kernel (int8, M = 100), split-K: C = acc + A @ B (int32 exactly; fp32 within
    summation error), the same bits on every launch."""
    import torch
    N, K = 1024, 8192
    say(f"tails 8-bit K-major decode acc {kind} M={M}")
    rng = np.random.default_rng(97)
    if kind == "i8":
        a, b = uniform_i8((M, K), 95), uniform_i8((K, N), 96)
        acc = rng.integers(-2 ** 20, 2 ** 20, size=(M, N)).astype(np.int32)
        da, tdt = to_device(a, gpu), None
        exact = (a.astype(np.int64) @ b.astype(np.int64) + acc).astype(np.int64)
    else:
        a, b = _codes8(rng, (M, K), "e4m3"), _codes8(rng, (K, N), "e4m3")
        acc = rng.standard_normal((M, N)).astype(np.float32)
        tdt = torch.float8_e4m3fn
        da = to_device(a, gpu).view(tdt)
        fa = oracle.e4m3_to_f32(a).astype(np.float64)
        fb = oracle.e4m3_to_f32(b).astype(np.float64)
        exact = fa @ fb + acc
    db = to_device(np.ascontiguousarray(b.T), gpu)
    db = (db if tdt is None else db.view(tdt)).t()
    dacc = to_device(acc, gpu)
    outs = []
    for _ in range(3):
        c = tx.dot(da, db, acc=dacc)
        torch.cuda.synchronize()
        outs.append(from_device(c))
    p = tx.plan_for(da, db, tx.tx_type(c), flags=tx.FLAG_ACCUMULATE)
    assert p.kernel == (tx.KERNEL_DECODE_F8 if M <= 64 else tx.KERNEL_DECODE_I8)
    assert p.split_k > 1 and p.desc.flags & tx.FLAG_B_KMAJOR
    if kind == "i8":
        assert np.array_equal(outs[0].astype(np.int64), exact)
    else:
        s = math.sqrt(K) * math.sqrt((fa ** 2).mean()) * math.sqrt((fb ** 2).mean())
        check_close(outs[0], exact, atol=ATOL, rtol=RTOL, scale=s, what="fp8 K-major acc")
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32))


@pytest.mark.parametrize("M,N,K,block", [
    (16, 8192, 8192, (0, 0, 0)), (1, 4096, 4096, (0, 0, 0)), (64, 1001, 999, (0, 0, 0)),
    (5, 300, 200, (0, 0, 0)), (17, 1001, 999, (256, 256, 128)), (300, 263, 391, (0, 0, 0)),
    (256, 8192, 8192, (0, 0, 0)), (100, 4100, 2049, (0, 0, 0)), (200, 1001, 999, (0, 0, 0)),
    (65, 130, 129, (0, 0, 0)), (700, 300, 200, (0, 0, 0)), (100, 300, 200, (256, 256, 128))])
def test_w8a8_kmajor_b(gpu, M, N, K, block):
    """W8A8 with the weight kept [N][K] (B a transposed view of junk-padded storage): the
    8-bit decode kernel's int8 form at M <= 48, the row decode kernel to M = 256 (slices of
    64 and 128 rows), the 256x256x128 tile (split-K) beyond or by name.  Bit-exact against the
    oracle (the same int32 sums and fp32 epilogue order)."""
    import torch
    say(f"tails W8A8 K-major B M={M} N={N} K={K} block={block}")
    a, b = uniform_i8((M, K), 101), uniform_i8((K, N), 102)
    sa_, sb_ = uniform_scales(M, 103), uniform_scales(N, 104)
    junk = np.random.default_rng(105)
    pa, _ = padded(a, 0)
    pa[:, K:] = junk.integers(-128, 128, size=pa[:, K:].shape)
    da = dev_view(pa, (M, K), gpu)
    db = _kmajor_b(b, 0, gpu, junk=junk)
    c = tx.dot(da, db, scale_a=to_device(sa_, gpu), scale_b=to_device(sb_, gpu),
               out_dtype=torch.bfloat16, block=block)
    torch.cuda.synchronize()
    _assert_kmajor_plan(da, db, c, tx.KERNEL_GEMM_I8, block, tx.SCALE_ROWCOL)
    ref = oracle.tiled_dot(a, b, a_type=oracle.I8, c_type=oracle.BF16, block=(64, 64, 64),
                           scale_mode=oracle.SCALE_ROWCOL, sa=sa_, sb=sb_)
    got = from_device(c)
    assert np.array_equal(got, ref), f"{np.count_nonzero(got != ref)} mismatches"


@pytest.mark.parametrize("M,N,K,out,block", [
    (16, 7168, 7168, "bf16", (0, 0, 0)), (1, 2048, 4096, "f32", (0, 0, 0)),
    (40, 1000, 1100, "bf16", (0, 0, 0)), (40, 1000, 1100, "f32", (256, 256, 128)),
    (300, 263, 391, "bf16", (0, 0, 0))])
def test_fp8_block_scaled_kmajor_b(gpu, M, N, K, out, block):
    """The block-scaled fp8 dot (config 4's form) with the weight kept [N][K], NaN codes in
    both operands' padding: the decode kernel at M <= 64, the 256 tile beyond or by name;
    against the oracle."""
    import torch
    say(f"tails fp8 block-scaled K-major B M={M} N={N} K={K} out={out} block={block}")
    qa, qb, sa, sb = fp8_block_inputs(M, N, K, 107)
    pa, _ = padded(qa, 0x7F)
    da = dev_view(pa, (M, K), gpu, torch.float8_e4m3fn)
    db = _kmajor_b(qb, 0x7F, gpu, torch.float8_e4m3fn)
    odt = torch.bfloat16 if out == "bf16" else torch.float32
    c = tx.dot(da, db, scale_a=to_device(sa, gpu), scale_b=to_device(sb, gpu), out_dtype=odt,
               block=block)
    torch.cuda.synchronize()
    _assert_kmajor_plan(da, db, c, tx.KERNEL_GEMM_F8, block, tx.SCALE_BLOCK128)
    ct = oracle.BF16 if out == "bf16" else oracle.F32
    ref = oracle.tiled_dot(qa, qb, a_type=oracle.F8E4M3, c_type=ct, block=(128, 128, 128),
                           scale_mode=oracle.SCALE_BLOCK128, sa=sa, sb=sb)
    got = from_device(c)
    if out == "bf16":
        got, ref = bits_to_f32(got, "bf16"), bits_to_f32(ref, "bf16")
    check_close(got, ref, atol=ATOL, rtol=RTOL, scale=math.sqrt(K), what="fp8 block K-major")
