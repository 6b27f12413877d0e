"""GPU parity: libmi355x_dot.so through the tx_dot C-ABI vs the CPU oracle.

Tolerances (north_star): int8 -> int32 bit-exact; fp16/bf16/fp8 with fp32
accumulation within |d| <= 1e-3 * s + 1e-2 * |ref|, s = 1 for inputs drawn
N(0,1)/sqrt(K) (outputs ~ 1/sqrt(K)), s = sqrt(K) for unnormalised inputs.
The oracle sums each K block in ascending k order; the MFMA sums in its own
order, so fp results agree to rounding, not bit for bit.
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


def run_16bit(gpu, M, N, K, kind, out_kind, block=(0, 0, 0), flags=0, seed=0, lda=None):
    import torch
    say(f"{kind}->{out_kind} M={M} N={N} K={K} block={block} flags={flags} lda={lda}")
    gen = normal_bf16 if kind == "bf16" else normal_f16
    a = gen((M, K if lda is None else lda), k_norm(K), 1 + seed)
    b = gen((K, N), k_norm(K), 2 + seed)
    da, db = to_device(a, gpu), to_device(b, gpu)
    tdt = torch.bfloat16 if kind == "bf16" else torch.float16
    da, db = da.view(tdt), db.view(tdt)
    if lda is not None:
        da = da[:, :K]
    out_dt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[out_kind]
    c = tx.dot(da, db, out_dtype=out_dt, block=block, flags=flags)
    torch.cuda.synchronize()
    got = from_device(c)
    return a[:, :K].copy(), b, got


def oracle_16bit(a, b, kind, out_kind, block, round_mode=oracle.ROUND_RNE):
    at = oracle.BF16 if kind == "bf16" else oracle.F16
    ct = {"f32": oracle.F32, "bf16": oracle.BF16, "f16": oracle.F16}[out_kind]
    return oracle.tiled_dot(a, b, a_type=at, c_type=ct, block=block, round_mode=round_mode)


def test_c1_fp16_512_block64(gpu):
    """Config 0: fp16 512^3, BLOCK 64x64x32, fp32 C."""
    a, b, got = run_16bit(gpu, 512, 512, 512, "f16", "f32", block=(64, 64, 32))
    ref = oracle_16bit(a, b, "f16", "f32", (64, 64, 32))
    err = check_close(got, ref, atol=ATOL, rtol=RTOL, what="fp16 512")
    # exact fp64 product as a second reference: fp32 rounding only
    exact = oracle.f16_to_f32(a).astype(np.float64) @ oracle.f16_to_f32(b).astype(np.float64)
    assert np.abs(got - exact).max() < 1e-5
    say(f"fp16 512 max|d|={err:.3g}")


def test_c2_bf16_4096(gpu):
    """Config 1: bf16 4096^3, bf16 C, the MFMA-bound headline case."""
    M = N = K = 4096
    a, b, got = run_16bit(gpu, M, N, K, "bf16", "bf16")
    p = tx.plan(tx.make_desc(M, N, K, tx.BF16, tx.BF16))
    blk = (p.desc.block_m, p.desc.block_n, p.desc.block_k)
    ref = oracle_16bit(a, b, "bf16", "bf16", blk)
    g, r = bits_to_f32(got, "bf16"), bits_to_f32(ref, "bf16")
    err = check_close(g, r, atol=ATOL, rtol=RTOL, what="bf16 4096")
    # against the interpreter's truncating cast too
    rtz = bits_to_f32(oracle_16bit(a, b, "bf16", "bf16", blk, oracle.ROUND_RTZ), "bf16")
    check_close(g, rtz, atol=ATOL, rtol=RTOL, what="bf16 4096 vs RTZ")
    # most outputs are bit-identical to the oracle's RNE bf16
    same = (got == ref).mean()
    assert same > 0.9, same
    say(f"bf16 4096 max|d|={err:.3g} max|d|*sqrt(K)={err * math.sqrt(K):.3g} identical={same:.4f}")


@pytest.mark.parametrize("M,N,K", [(4096, 4096, 4000), (4000, 4000, 4000)])
def test_c3_loop_split_tail_and_edges(gpu, M, N, K):
    """Config 2: K-tail peeled from the main loop (K=4000 = 62*64 + 32), edge tiles."""
    p = tx.plan(tx.make_desc(M, N, K, tx.BF16, tx.BF16))
    assert (p.k_split, p.k_main_steps, p.k_tail) == (3968, 62, 32)
    a, b, got = run_16bit(gpu, M, N, K, "bf16", "bf16")
    blk = (p.desc.block_m, p.desc.block_n, p.desc.block_k)
    ref = oracle_16bit(a, b, "bf16", "bf16", blk)
    err = check_close(bits_to_f32(got, "bf16"), bits_to_f32(ref, "bf16"), atol=ATOL, rtol=RTOL,
                      what=f"bf16 {M}x{N}x{K}")
    say(f"tail {M}x{N}x{K} max|d|={err:.3g}")


def test_loop_split_equals_all_masked(gpu):
    """Peeling changes which loads test bounds, not the arithmetic: bit-identical."""
    M, N, K = 1000, 1000, 1000
    _, _, split = run_16bit(gpu, M, N, K, "bf16", "f32", block=(128, 128, 64), seed=5)
    _, _, masked = run_16bit(gpu, M, N, K, "bf16", "f32", block=(128, 128, 64), seed=5,
                             flags=tx.FLAG_NO_LOOP_SPLIT)
    assert np.array_equal(split, masked)


@pytest.mark.parametrize("M,N,K,block,kind,out", [
    (64, 64, 32, (64, 64, 32), "f16", "f32"),
    (1, 8, 8, (64, 64, 32), "bf16", "f32"),
    (33, 72, 24, (64, 64, 32), "f16", "f16"),
    (257, 264, 136, (128, 128, 64), "bf16", "bf16"),
    (300, 520, 200, (256, 256, 64), "bf16", "f32"),
    (128, 128, 8, (128, 128, 64), "f16", "f32"),
])
def test_16bit_edges(gpu, M, N, K, block, kind, out):
    a, b, got = run_16bit(gpu, M, N, K, kind, out, block=block, seed=M)
    ref = oracle_16bit(a, b, kind, out, block)
    check_close(bits_to_f32(got, out), bits_to_f32(ref, out), atol=ATOL, rtol=RTOL,
                what=f"{kind} {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K,kind,out", [(1024, 1024, 1024, "bf16", "bf16"),
                                             (300, 520, 200, "bf16", "f32"),
                                             (256, 256, 64, "f16", "f32"),
                                             (4096, 4096, 4000, "bf16", "bf16"),
                                             (1000, 1000, 1000, "f16", "f16")])
def test_b_kmajor(gpu, M, N, K, kind, out):
    """q @ k.T: B passed as the transpose of a row-major [N, K] tensor."""
    import torch
    say(f"K-major B {kind}->{out} M={M} N={N} K={K}")
    gen = normal_bf16 if kind == "bf16" else normal_f16
    a = gen((M, K), k_norm(K), M + 1)
    bt = gen((N, K), k_norm(K), N + 2)                     # [N, K] row-major
    tdt = torch.bfloat16 if kind == "bf16" else torch.float16
    odt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[out]
    da = to_device(a, gpu).view(tdt)
    db = to_device(bt, gpu).view(tdt).t()                  # [K, N] view, K-major
    assert db.stride() == (1, K)
    c = tx.dot(da, db, out_dtype=odt)
    torch.cuda.synchronize()
    got = from_device(c)
    at = oracle.BF16 if kind == "bf16" else oracle.F16
    ct = {"bf16": oracle.BF16, "f16": oracle.F16, "f32": oracle.F32}[out]
    ref = oracle.tiled_dot(a, np.ascontiguousarray(bt.T), a_type=at, c_type=ct,
                           block=(256, 256, 64), round_mode=oracle.ROUND_RNE)
    if out == "f32":
        check_close(got, ref, atol=ATOL, rtol=RTOL, what="K-major B")
    else:
        check_close(bits_to_f32(got, out), bits_to_f32(ref, out), atol=ATOL, rtol=RTOL,
                    what="K-major B")


def test_strided_a(gpu):
    a, b, got = run_16bit(gpu, 200, 256, 192, "bf16", "f32", block=(128, 128, 64), lda=256)
    ref = oracle_16bit(a, b, "bf16", "f32", (128, 128, 64))
    check_close(got, ref, atol=ATOL, rtol=RTOL, what="strided A")


def test_unaligned_row_stride(gpu):
    """A row stride that is not a multiple of 16 bytes is rejected at plan time (the
    kernels read 16-byte chunks); dot() copies such an operand into padded rows
    itself, and the result stays bit-exact (int8 -> int32, K = 200)."""
    import torch
    say("unaligned row stride")
    with pytest.raises(tx.TxError) as e:
        tx.plan(tx.make_desc(5, 272, 200, tx.I8, tx.I32, lda=200))
    assert e.value.code == tx.ERR_INVALID
    a = uniform_i8((5, 200), 121)
    b = uniform_i8((200, 272), 122)
    c = tx.dot(to_device(a, gpu), to_device(b, gpu), out_dtype=torch.int32)
    torch.cuda.synchronize()
    assert np.array_equal(from_device(c), a.astype(np.int64) @ b.astype(np.int64))


def test_k_zero_and_empty(gpu):
    import torch
    say("K=0 and empty outputs")
    a = torch.zeros((64, 0), dtype=torch.bfloat16, device=gpu)
    b = torch.zeros((0, 64), dtype=torch.bfloat16, device=gpu)
    c = tx.dot(a, b, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert (c == 0).all()
    e = tx.dot(torch.zeros((0, 64), dtype=torch.bfloat16, device=gpu),
               torch.zeros((64, 64), dtype=torch.bfloat16, device=gpu), out_dtype=torch.float32)
    assert e.shape == (0, 64)


# ----------------------------------------------------------------------------- int8


def run_w8a8(gpu, M, N, K, seed=0, block=(0, 0, 0)):
    import torch
    say(f"w8a8 M={M} N={N} K={K} block={block}")
    a = uniform_i8((M, K), 1 + seed)
    b = uniform_i8((K, N), 2 + seed)
    sa = uniform_scales(M, 3 + seed)
    sb = uniform_scales(N, 4 + seed)
    c = tx.dot(to_device(a, gpu), to_device(b, gpu), scale_a=to_device(sa, gpu),
               scale_b=to_device(sb, gpu), out_dtype=torch.bfloat16, block=block)
    torch.cuda.synchronize()
    return a, b, sa, sb, from_device(c)


@pytest.mark.parametrize("M", [1, 16, 64, 256])
def test_c4_w8a8_decode(gpu, M):
    """Config 3: int8 W8A8, N=K=8192: int32 exact, so the bf16 output is bit-exact."""
    N = K = 8192
    a, b, sa, sb, got = run_w8a8(gpu, M, N, K)
    ref = oracle.tiled_dot(a, b, a_type=oracle.I8, c_type=oracle.BF16, block=(64, 256, 128),
                           scale_mode=oracle.SCALE_ROWCOL, sa=sa, sb=sb, round_mode=oracle.ROUND_RNE)
    mism = np.flatnonzero(got != ref)
    assert mism.size == 0, f"{mism.size} mismatches, first at {np.unravel_index(mism[0], got.shape)}"


@pytest.mark.parametrize("M,N,K", [(5, 272, 208), (16, 256, 64), (40, 8208, 1008), (3, 16, 4160),
                                   (64, 512, 16), (17, 4096, 2080), (65, 8208, 1008),
                                   (100, 4096, 2080), (130, 272, 4160), (200, 1024, 64),
                                   (256, 8192, 1024), (300, 1024, 1040), (512, 8192, 2048)])
def test_w8a8_decode_edges(gpu, M, N, K):
    """Decode shapes at the planner's tiles: waves splitting K up to M = 48, the row kernel's
    slices of 64 and 128 rows beyond (M = 49 .. 256), the 256x256x128 tile with split-K past
    it."""
    a, b, sa, sb, got = run_w8a8(gpu, M, N, K, seed=M)
    ref = oracle.tiled_dot(a, b, a_type=oracle.I8, c_type=oracle.BF16, block=(64, 64, 64),
                           scale_mode=oracle.SCALE_ROWCOL, sa=sa, sb=sb, round_mode=oracle.ROUND_RNE)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("M,N,K,bm", [(256, 8192, 8192, 256), (256, 8192, 8192, 128),
                                      (192, 4096, 8192, 128), (128, 8192, 8192, 128),
                                      (65, 8208, 1008, 128), (100, 4096, 2080, 256),
                                      (130, 272, 4160, 256), (200, 1024, 64, 256),
                                      (255, 1000, 2000, 256), (192, 8200, 8190, 256),
                                      (129, 16, 16, 128), (64, 8192, 8192, 64),
                                      (16, 8192, 8192, 64), (40, 4096, 2080, 64),
                                      (130, 272, 4160, 64), (1, 8200, 1000, 64),
                                      (384, 4096, 2048, 256), (300, 1000, 3000, 256),
                                      (700, 8192, 512, 256), (1024, 2048, 1024, 64)])
def test_w8a8_row_kernel(gpu, M, N, K, bm):
    """The row-parallel decode tile (block (64 | 128 | 256, 128, 128): every wave takes every
    128-row K batch of its strip, B staged once per slice in a shared ring), split-K included:
    bit-exact, ragged M, N and K included."""
    a, b, sa, sb, got = run_w8a8(gpu, M, N, K, seed=M + bm, block=(bm, 128, 128))
    ref = oracle.tiled_dot(a, b, a_type=oracle.I8, c_type=oracle.BF16, block=(64, 64, 64),
                           scale_mode=oracle.SCALE_ROWCOL, sa=sa, sb=sb, round_mode=oracle.ROUND_RNE)
    mism = np.flatnonzero(got != ref)
    assert mism.size == 0, f"{mism.size} mismatches, first at {np.unravel_index(mism[0], got.shape)}"


def test_w8a8_row_kernel_shares_workspace(gpu):
    """Row-kernel and sliced launches of different shapes on one cached workspace: the counters
    each leaves at zero serve the next."""
    for M, N, K, bm in ((256, 8192, 8192, 256), (16, 8192, 8192, 0), (128, 8192, 8192, 128),
                        (256, 8192, 8192, 64), (256, 4096, 8192, 256)):
        a, b, sa, sb, got = run_w8a8(gpu, M, N, K, seed=M + N + bm,
                                     block=(bm, 128, 128 if bm > 64 else 64) if bm else (0, 0, 0))
        ref = oracle.tiled_dot(a, b, a_type=oracle.I8, c_type=oracle.BF16, block=(64, 256, 128),
                               scale_mode=oracle.SCALE_ROWCOL, sa=sa, sb=sb)
        assert np.array_equal(got, ref), f"M={M} N={N} K={K} block_m={bm}"


def test_w8a8_workspace_across_shapes(gpu):
    """One cached workspace serves decode launches of different shapes: a launch with more row
    slices or strips than the last must not read the last one's partials as arrival counters."""
    for M, N, K in ((16, 8192, 8192), (128, 8192, 8192), (100, 16384, 4096), (16, 8192, 8192),
                    (128, 8192, 8192)):
        a, b, sa, sb, got = run_w8a8(gpu, M, N, K, seed=M + N)
        ref = oracle.tiled_dot(a, b, a_type=oracle.I8, c_type=oracle.BF16, block=(64, 256, 128),
                               scale_mode=oracle.SCALE_ROWCOL, sa=sa, sb=sb)
        assert np.array_equal(got, ref), f"M={M} N={N} K={K}"


def test_w8a8_repeat_launches(gpu):
    """The arrival counters carry over between launches: repeat, then change shape."""
    for M, N, K in ((16, 8192, 8192), (16, 8192, 8192), (7, 4096, 2048), (16, 8192, 8192)):
        a, b, sa, sb, got = run_w8a8(gpu, M, N, K, seed=11)
        ref = oracle.tiled_dot(a, b, a_type=oracle.I8, c_type=oracle.BF16, block=(64, 256, 128),
                               scale_mode=oracle.SCALE_ROWCOL, sa=sa, sb=sb)
        assert np.array_equal(got, ref)


@pytest.mark.parametrize("M,N,K,block", [(300, 304, 256, (128, 128, 128)),
                                          (256, 512, 1000 - 1000 % 16, (256, 256, 128)),
                                          (2, 16, 16, (128, 128, 128)),
                                          (2, 4096, 1024, (0, 0, 0)), (64, 512, 256, (0, 0, 0))])
def test_int8_gemm_int32_exact(gpu, M, N, K, block):
    import torch
    say(f"int8 gemm i32 M={M} N={N} K={K} block={block}")
    a = uniform_i8((M, K), 21)
    b = uniform_i8((K, N), 22)
    c = tx.dot(to_device(a, gpu), to_device(b, gpu), out_dtype=torch.int32, block=block)
    torch.cuda.synchronize()
    got = from_device(c)
    exact = a.astype(np.int64) @ b.astype(np.int64)
    assert np.array_equal(got.astype(np.int64), exact)


# ----------------------------------------------------------------------------- fp8


@pytest.mark.parametrize("M,N,K", [(2048, 7168, 7168), (200, 384, 640), (130, 250 + 6, 384)])
def test_c5_fp8_block_scaled(gpu, M, N, K):
    """Config 4: fp8 e4m3, 1x128 A-group and 128x128 B-block fp32 scales."""
    import torch
    say(f"fp8 block-scaled M={M} N={N} K={K}")
    qa, qb, sa, sb = fp8_block_inputs(M, N, K, 7)
    c = tx.dot(to_device(qa, gpu), to_device(qb, gpu), scale_a=to_device(sa, gpu),
               scale_b=to_device(sb, gpu), out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    got = bits_to_f32(from_device(c), "bf16")
    ref = bits_to_f32(oracle.tiled_dot(qa, qb, a_type=oracle.F8E4M3, c_type=oracle.BF16,
                                       block=(128, 128, 128), scale_mode=oracle.SCALE_BLOCK128,
                                       sa=sa, sb=sb), "bf16")
    err = check_close(got, ref, atol=ATOL, rtol=RTOL, scale=math.sqrt(K), what="fp8")
    say(f"fp8 {M}x{N}x{K} max|d|={err:.3g}")


@pytest.mark.parametrize("kind,out", [("i8", "rowcol"), ("f8", "f32"), ("f8", "block_f32"),
                                      ("f8", "block_bf16")])
@pytest.mark.parametrize("M,N,K", [(512, 512, 1024), (300, 272, 400), (16, 1024, 256)])
@pytest.mark.parametrize("blk", [(256, 256, 128), (256, 224, 128), (128, 128, 128)])
def test_8bit_tile_epilogues(gpu, kind, out, M, N, K, blk):
    """Each epilogue of the 8-bit tile kernels, whole and edge tiles (M, N
    not multiples of the tile; K not a multiple of 128: a masked last step).
    Unscaled fp8 uses full-range e4m3 values (|q| up to 448), whose running
    sums cancel to much smaller results."""
    import torch
    say(f"8-bit tile {kind}/{out} M={M} N={N} K={K} block={blk}")
    if kind == "i8":
        a = uniform_i8((M, K), 31)
        b = uniform_i8((K, N), 32)
        sa = uniform_scales(M, 33)
        sb = uniform_scales(N, 34)
        c = tx.dot(to_device(a, gpu), to_device(b, gpu), scale_a=to_device(sa, gpu),
                   scale_b=to_device(sb, gpu), out_dtype=torch.bfloat16, block=blk)
        torch.cuda.synchronize()
        ref = oracle.tiled_dot(a, b, a_type=oracle.I8, c_type=oracle.BF16, block=(64, 64, 64),
                               scale_mode=oracle.SCALE_ROWCOL, sa=sa, sb=sb,
                               round_mode=oracle.ROUND_RNE)
        assert np.array_equal(from_device(c), ref)
        return
    qa, qb, sa, sb = fp8_block_inputs(M, N, K, 35)
    norm = math.sqrt(K)
    if out == "f32":
        c = tx.dot(to_device(qa, gpu), to_device(qb, gpu), out_dtype=torch.float32, block=blk)
        ct, sm, kw = oracle.F32, oracle.SCALE_NONE, {}
        # Unscaled codes: normalise by the operands' RMS as well as sqrt(K).
        rms = lambda q: float(np.sqrt(np.mean(oracle.e4m3_to_f32(q).astype(np.float64) ** 2)))
        norm *= rms(qa) * rms(qb)
    else:
        odt = torch.float32 if out == "block_f32" else torch.bfloat16
        c = tx.dot(to_device(qa, gpu), to_device(qb, gpu), scale_a=to_device(sa, gpu),
                   scale_b=to_device(sb, gpu), out_dtype=odt, block=blk)
        ct = oracle.F32 if out == "block_f32" else oracle.BF16
        sm, kw = oracle.SCALE_BLOCK128, dict(sa=sa, sb=sb)
    torch.cuda.synchronize()
    got = from_device(c)
    ref = oracle.tiled_dot(qa, qb, a_type=oracle.F8E4M3, c_type=ct, block=(128, 128, 128),
                           scale_mode=sm, **kw)
    if ct == oracle.BF16:
        got, ref = bits_to_f32(got, "bf16"), bits_to_f32(ref, "bf16")
    err = check_close(got, ref, atol=ATOL, rtol=RTOL, scale=norm, what=f"fp8 {out}")
    say(f"fp8 {out} {M}x{N}x{K} max|d|={err:.3g} (normalised {err / norm:.3g})")


# ----------------------------------------------------------------------------- golden fixtures

GOLDEN_TILE = {"f16": (64, 64, 32), "bf16": (128, 128, 64), "i8": (128, 128, 128),
               "f8e4m3": (128, 128, 128), "f8e5m2": (256, 256, 128)}


@pytest.mark.parametrize("name", ["c1_fp16_512", "fp16_f32_edges_exact", "fp16_f16_rne_exact",
                                  "bf16_bf16_rtz_exact", "bf16_f32_normal", "int8_i32",
                                  "w8a8_rowcol_rtz", "fp8_block128_f32_exact",
                                  "fp8_block128_bf16_normal", "fp8e5_f32_exact",
                                  "fp8e4e5_f32_exact", "fp8e5_f32_normal"])
def test_golden_fixture_on_gpu(gpu, name):
    """The interpreter's fixtures through the HIP path.

    Exact fixtures (every fp32 partial sum exact): the GPU output equals the
    oracle's bit for bit, and where the interpreter truncated to bf16, the
    GPU's fp32 accumulator truncated gives the fixture's bits.  Others: within
    the north_star tolerance of the fixture."""
    golden_on_gpu(gpu, name, None)


@pytest.mark.parametrize("tile", [(256, 256, 128), (256, 224, 128)])
@pytest.mark.parametrize("name", ["int8_i32", "fp8_block128_f32_exact", "fp8_block128_bf16_normal"])
def test_golden_fixture_256_tile(gpu, name, tile):
    """The 8-bit fixtures through the 256-row tile kernels (8 waves)."""
    golden_on_gpu(gpu, name, tile)


@pytest.mark.parametrize("name", ["c1_fp16_512", "fp16_f32_edges_exact", "fp16_f16_rne_exact",
                                  "bf16_bf16_rtz_exact", "bf16_f32_normal"])
def test_golden_fixture_b_kmajor(gpu, name):
    """The 16-bit fixtures with B stored K-major ([N, K] row-major)."""
    golden_on_gpu(gpu, name, (256, 256, 64), b_kmajor=True)


def golden_on_gpu(gpu, name, tile, b_kmajor=False):
    import os
    import torch
    from test_oracle_cpu import GOLDEN, OR_TYPE, fixture_output, load_fixture
    say(f"golden {name} tile={tile}")
    f = load_fixture(os.path.join(GOLDEN, name + ".npz"))
    at, ct = str(f["a_type"]), str(f["c_type"])
    bt = str(f.get("b_type", at))
    tdt = {"f16": torch.float16, "bf16": torch.bfloat16, "i8": torch.int8,
           "f8e4m3": torch.float8_e4m3fn, "f8e5m2": torch.float8_e5m2}
    odt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16,
           "i32": torch.int32}[ct]
    view = {"f16": torch.int16, "bf16": torch.int16, "f8e4m3": torch.uint8, "f8e5m2": torch.uint8,
            "i8": torch.int8}
    da = to_device(f["a"], gpu).view(view[at]).view(tdt[at])
    if b_kmajor:
        db = to_device(np.ascontiguousarray(f["b"].T), gpu).view(view[bt]).view(tdt[bt]).t()
    else:
        db = to_device(f["b"], gpu).view(view[bt]).view(tdt[bt])
    kw = {}
    if "sa" in f:
        kw = dict(scale_a=to_device(f["sa"], gpu), scale_b=to_device(f["sb"], gpu))
    blk = GOLDEN_TILE[bt if bt == "f8e5m2" else at] if name != "c1_fp16_512" else (64, 64, 32)
    if name == "w8a8_rowcol_rtz":
        blk = (0, 0, 0)  # M = 5: the decode kernel
    if tile is not None:
        blk = tile
    c = tx.dot(da, db, out_dtype=odt, block=blk, **kw)
    c32 = tx.dot(da, db, out_dtype=torch.float32, block=blk, **kw) if ct == "bf16" and at != "i8" \
        else None
    torch.cuda.synchronize()
    got = from_device(c)
    sm = {0: oracle.SCALE_NONE, 1: oracle.SCALE_ROWCOL, 2: oracle.SCALE_BLOCK128}[int(f["epi"])]
    oblk = blk if blk != (0, 0, 0) else (64, 64, 64)
    ref = oracle.tiled_dot(f["a"], f["b"], a_type=OR_TYPE[at], c_type=OR_TYPE[ct], block=oblk,
                           scale_mode=sm, sa=f.get("sa"), sb=f.get("sb"),
                           round_mode=oracle.ROUND_RNE, b_type=OR_TYPE[bt])
    if bool(f["exact"]) and at == "f8e4m3" and sm == oracle.SCALE_BLOCK128 and blk[0] == 256:
        # (both 256-row tiles: 256x256 and 256x224)
        # The 256-wide fp8 tile applies a block's scales as one fma(part,
        # sa*sb, acc) (two roundings) where the interpreter rounds
        # part*sa, then *sb, then the sum (three): per K block, the two
        # differ by at most 3 units in the last place of |part*sa*sb|, and
        # the running sums by one more of the accumulator's.
        fa = np.abs(oracle.e4m3_to_f32(f["a"]).astype(np.float64))
        fb = np.abs(oracle.e4m3_to_f32(f["b"]).astype(np.float64))
        K, N = fa.shape[1], fb.shape[1]
        nkb = (K + 127) // 128
        S = np.zeros((fa.shape[0], N))
        for kb in range(nkb):
            part = fa[:, kb * 128:(kb + 1) * 128] @ fb[kb * 128:(kb + 1) * 128]
            S += part * f["sa"][:, kb:kb + 1] * np.repeat(f["sb"][kb], 128)[:N]
        bound = (nkb + 4) * 2.0 ** -24 * S
        d = np.abs(got.astype(np.float64) - ref.astype(np.float64))
        assert (d <= bound).all(), f"{np.count_nonzero(d > bound)} beyond the rounding bound"
        say(f"golden {name}: {np.count_nonzero(d)} of {d.size} differ, max d/bound "
            f"{(d / np.maximum(bound, 1e-300)).max():.3g}")
        return
    if bool(f["exact"]):
        assert np.array_equal(got, ref), f"{np.count_nonzero(got != ref)} elements differ"
        if ct == "bf16" and c32 is not None:
            trunc = (from_device(c32).view(np.uint32) >> 16).astype(np.uint16)
            g, w = fixture_output(f, trunc)
            assert np.array_equal(g, w)
        return
    g, w = fixture_output(f, got)
    K = int(f["K"])
    scale = math.sqrt(K) if at in ("f8e4m3", "f8e5m2") else 1.0
    check_close(bits_to_f32(g, ct), bits_to_f32(w, ct), atol=ATOL, rtol=RTOL, scale=scale,
                what=f"golden {name}")


@pytest.mark.parametrize("fa,fb", [("e5m2", "e5m2"), ("e4m3", "e5m2"), ("e5m2", "e4m3")])
@pytest.mark.parametrize("M,N,K", [(512, 512, 1024), (300, 272, 400), (16, 1024, 256)])
def test_fp8_e5m2_dot(gpu, fa, fb, M, N, K):
    """tt.dot of fp8 operands with e5m2 on a side (the tutorial's p . v with
    fp8e5 p), fp32 C, on the 256x256 8-bit tile: edges, a K tail, small M.
    Finite codes across the whole range; tolerance normalised by the
    operands' RMS (the MFMA's fixed-point group sums)."""
    import torch
    say(f"fp8 {fa}x{fb} M={M} N={N} K={K}")
    rng = np.random.default_rng(M + N + K)

    def codes(shape, f):
        c = rng.integers(0, 256, size=shape).astype(np.uint8)
        if f == "e5m2":
            return np.where((c & 0x7C) == 0x7C, c & 0x83, c).astype(np.uint8)
        return np.where((c & 0x7F) == 0x7F, c & 0xF0, c).astype(np.uint8)
    a, b = codes((M, K), fa), codes((K, N), fb)
    tdt = {"e4m3": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}
    otype = {"e4m3": oracle.F8E4M3, "e5m2": oracle.F8E5M2}
    da = to_device(a, gpu).view(tdt[fa])
    db = to_device(b, gpu).view(tdt[fb])
    p = tx.plan_for(da, db, tx.F32)
    assert p.kernel == (tx.KERNEL_DECODE_F8 if M <= 64 else tx.KERNEL_GEMM_F8)
    c = tx.dot(da, db, out_dtype=torch.float32)
    torch.cuda.synchronize()
    got = from_device(c)
    ref = oracle.tiled_dot(a, b, a_type=otype[fa], b_type=otype[fb], c_type=oracle.F32,
                           block=(256, 256, 128))
    dec = lambda q, f: (oracle.e4m3_to_f32(q) if f == "e4m3"
                        else oracle.f16_to_f32(q.astype(np.uint16) << 8)).astype(np.float64)
    rms = lambda q, f: float(np.sqrt(np.mean(dec(q, f) ** 2)))
    err = check_close(got, ref, atol=ATOL, rtol=RTOL, scale=math.sqrt(K) * rms(a, fa) * rms(b, fb),
                      what=f"fp8 {fa}x{fb}")
    say(f"fp8 {fa}x{fb} {M}x{N}x{K}: max|d|={err:.3g}")


# ----------------------------------------------------------------------------- accumulate
@pytest.mark.parametrize("kind,M,N,K", [("bf16", 512, 512, 1024), ("bf16", 300, 272, 416),
                                        ("f16", 256, 512, 4000), ("i8", 512, 256, 1024),
                                        ("i8", 96, 160, 640), ("f8", 512, 512, 512),
                                        ("bf16", 128, 256, 0)])
def test_accumulate(gpu, kind, M, N, K):
    """tl.dot(a, b, acc): TX_FLAG_ACCUMULATE stores fl(C + sum) -- bit for bit
    the non-accumulating result plus C in one fp32 addition (int32: exactly),
    on the 256x256 tiles, the small register-staged tiles and K = 0."""
    import torch
    say(f"accumulate {kind} {M}x{N}x{K}")
    g = torch.Generator(device=gpu)
    g.manual_seed(M + N + K)
    if kind == "i8":
        a = torch.randint(-127, 128, (M, K), generator=g, device=gpu, dtype=torch.int8)
        b = torch.randint(-127, 128, (K, N), generator=g, device=gpu, dtype=torch.int8)
        c0 = torch.randint(-2 ** 20, 2 ** 20, (M, N), generator=g, device=gpu, dtype=torch.int32)
        odt = torch.int32
    else:
        dt = {"bf16": torch.bfloat16, "f16": torch.float16, "f8": torch.float8_e4m3fn}[kind]
        a = torch.randn((M, K), generator=g, device=gpu).to(dt)
        b = torch.randn((K, N), generator=g, device=gpu).to(dt)
        c0 = torch.randn((M, N), generator=g, device=gpu) * 3
        odt = torch.float32
    c0_host = from_device(c0).copy()
    plain = tx.dot(a, b, out_dtype=odt)
    got = tx.dot(a, b, out_dtype=odt, acc=c0)
    torch.cuda.synchronize()
    want = (from_device(plain) + from_device(c0)).astype(np.int32 if odt == torch.int32
                                                          else np.float32)
    g_ = from_device(got)
    assert np.array_equal(g_.view(np.int32), want.view(np.int32)), \
        f"max |d| {np.abs(g_.astype(np.float64) - want).max()}"
    assert np.array_equal(from_device(c0).view(np.int32), c0_host.view(np.int32)), \
        "acc itself was written"


@pytest.mark.parametrize("lhs_fmt,rhs_fmt", [("e4m3", "e4m3"), ("e2m1", "e2m1"), ("bf16", "e2m1")])
def test_dot_scaled_accumulate(gpu, lhs_fmt, rhs_fmt):
    """tl.dot_scaled(..., acc): acc + the dot, bit for bit the plain result
    plus acc in one fp32 addition."""
    import torch
    say(f"dot_scaled acc {lhs_fmt} x {rhs_fmt}")
    M, N, K = 320, 256, 512
    rng = np.random.default_rng(9)
    def operand(fmt, rows, cols, kdim):
        if fmt == "bf16":
            return torch.from_numpy(rng.standard_normal((rows, cols)).astype(np.float32)) \
                .to(torch.bfloat16).to(gpu), None
        c = rng.integers(0, 16 if fmt == "e2m1" else 0x70, size=(rows, cols)).astype(np.uint8)
        if fmt == "e2m1":
            c = (c[:, 0::2] | (c[:, 1::2] << 4)) if kdim == 1 else (c[0::2] | (c[1::2] << 4))
        return to_device(np.ascontiguousarray(c.astype(np.uint8)), gpu), None
    a, _ = operand(lhs_fmt, M, K, 1)
    b, _ = operand(rhs_fmt, K, N, 0)
    sa = None if lhs_fmt == "bf16" else to_device(rng.integers(120, 134, (M, K // 32)).astype(np.uint8), gpu)
    sb = None if rhs_fmt == "bf16" else to_device(rng.integers(120, 134, (N, K // 32)).astype(np.uint8), gpu)
    acc = torch.from_numpy(rng.standard_normal((M, N)).astype(np.float32)).to(gpu)
    plain = tx.dot_scaled(a, sa, lhs_fmt, b, sb, rhs_fmt)
    got = tx.dot_scaled(a, sa, lhs_fmt, b, sb, rhs_fmt, acc=acc)
    torch.cuda.synchronize()
    want = (from_device(plain) + from_device(acc)).astype(np.float32)
    assert np.array_equal(from_device(got).view(np.int32), want.view(np.int32))


def test_e4m3_max_codes_are_nan(gpu):
    """e4m3 codes 0x7F / 0xFF.  gfx950's MFMA reads them as NaN, as OCP e4m3fn
    (Triton's fp8e4nv, torch.float8_e4m3fn) defines them; the Triton
    interpreter's generic converter decodes them as +-480
    (T:runtime/interpreter.py:202-263), which the interpreter fixture and the
    oracle reproduce.  The product keeps the hardware's reading: every output
    whose row of A or column of B holds such a code is NaN, and every other
    output equals the interpreter's bit for bit (the fixture is dyadic)."""
    import os

    import torch
    from test_oracle_cpu import GOLDEN, load_fixture
    f = load_fixture(os.path.join(GOLDEN, "fp8e4m3_maxcode_f32_exact.npz"))
    a, b = f["a"], f["b"]
    say("e4m3 max codes")
    c = tx.dot(to_device(a, gpu).view(torch.float8_e4m3fn),
               to_device(b, gpu).view(torch.float8_e4m3fn), out_dtype=torch.float32)
    torch.cuda.synchronize()
    got = from_device(c)
    bad_rows = ((a & 0x7F) == 0x7F).any(axis=1)
    bad_cols = ((b & 0x7F) == 0x7F).any(axis=0)
    poisoned = bad_rows[:, None] | bad_cols[None, :]
    assert bad_rows.sum() == 3 and bad_cols.sum() == 1
    assert np.isnan(got[poisoned]).all()
    assert np.array_equal(got[~poisoned], f["c"][~poisoned])
    # the interpreter itself (and the oracle) read +-480: finite everywhere
    assert np.isfinite(f["c"]).all()
