"""tx_dot_launch_noalloc: the launch entry point that allocates nothing.

Its kernels are tx_dot_launch's; only the workspace differs (the library's
static per-GPU scratch array instead of the caller's buffer).  So its output
must equal tx_dot_launch's bit for bit on the same inputs, for the kernels
that use scratch: the decode kernels (split-K counters and partials: W8A8
int32, 16-bit fp32) and the MX x bf16 upcast (the bf16 operand).  Two calls in a row, the second
smaller, check that a call does not depend on what the previous one left in
the shared array; the decode results are also checked against the oracle
(int32 exact, so bit-exact bf16).
"""
import ctypes

import numpy as np
import pytest

import oracle
import triton_ext_amd as tx
from dotcase import from_device, say, to_device, uniform_i8, uniform_scales

pytestmark = pytest.mark.gpu


def _launch(fn_name, plan, a, b, c, sa, sb, ws=None):
    import torch
    L = tx.load()
    stream = torch.cuda.current_stream().cuda_stream
    ptrs = (ctypes.byref(plan), a.data_ptr(), b.data_ptr(), c.data_ptr(),
            None if sa is None else sa.data_ptr(), None if sb is None else sb.data_ptr())
    if fn_name == "noalloc":
        rc = L.tx_dot_launch_noalloc(*ptrs, stream)
    else:
        rc = L.tx_dot_launch(*ptrs, None if ws is None else ws.data_ptr(),
                             0 if ws is None else ws.numel(), stream)
    assert rc == tx.OK, L.tx_get_last_error().decode()


def _w8a8(gpu, M, N, K, seed):
    import torch
    say(f"noalloc W8A8 M={M} N={N} K={K} seed={seed}")
    a = uniform_i8((M, K), seed)
    b = uniform_i8((K, N), seed + 1)
    sa = uniform_scales(M, seed + 2)
    sb = uniform_scales(N, seed + 3)
    da, db, dsa, dsb = (to_device(x, gpu) for x in (a, b, sa, sb))
    plan = tx.plan(tx.make_desc(M, N, K, tx.I8, tx.BF16, scale_mode=tx.SCALE_ROWCOL))
    assert plan.kernel == tx.KERNEL_DECODE_I8
    c_ref = torch.empty((M, N), dtype=torch.bfloat16, device=gpu)
    c_new = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu)
    ws = torch.zeros(max(int(plan.workspace_bytes), 1), dtype=torch.uint8, device=gpu)
    _launch("plain", plan, da, db, c_ref, dsa, dsb, ws)
    _launch("noalloc", plan, da, db, c_new, dsa, dsb)
    torch.cuda.synchronize()
    ref, got = from_device(c_ref), from_device(c_new)
    assert np.array_equal(got, ref), f"{np.count_nonzero(got != ref)} elements differ"
    orc = oracle.tiled_dot(a, b, a_type=oracle.I8, c_type=oracle.BF16, block=(64, 256, 128),
                           scale_mode=oracle.SCALE_ROWCOL, sa=sa, sb=sb)
    assert np.array_equal(got, orc)
    return plan


def test_noalloc_w8a8_two_calls(gpu):
    """Split-K decode, then a smaller one (fewer strips, another split) on the same scratch."""
    p1 = _w8a8(gpu, 16, 8192, 8192, 21)
    p2 = _w8a8(gpu, 5, 2048, 4096, 22)
    assert p1.split_k > 1 and p2.split_k > 1 and p2.workspace_bytes < p1.workspace_bytes
    _w8a8(gpu, 16, 8192, 8192, 23)  # and back: the counters were left at zero


def test_noalloc_row_kernel_between_split_calls(gpu):
    """The row-slice decode kernel (64- and 128-row slices, split-K) on the same scratch as the
    K-split kernel: each leaves the shared counters at zero for the next."""
    p1 = _w8a8(gpu, 256, 2048, 4096, 51)
    p2 = _w8a8(gpu, 100, 4096, 2048, 52)
    assert (p1.desc.block_m, p1.desc.block_k) == (128, 128) and p1.split_k > 1
    assert (p2.desc.block_m, p2.desc.block_k) == (64, 128) and p2.split_k > 1
    _w8a8(gpu, 16, 8192, 8192, 53)


def _mx_bf16(gpu, M, N, K, seed):
    import torch
    say(f"noalloc MX x bf16 M={M} N={N} K={K} seed={seed}")
    g = torch.Generator(device=gpu)
    g.manual_seed(seed)
    a = torch.randn((M, K), generator=g, device=gpu).to(torch.bfloat16)
    codes = torch.randint(0, 256, (K, N), generator=g, device=gpu, dtype=torch.int32)
    codes = codes.to(torch.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0  # no e4m3 NaN codes
    scales = torch.randint(120, 134, (N, K // 32), generator=g, device=gpu,
                           dtype=torch.int32).to(torch.uint8)
    plan = tx.plan(tx.make_desc(M, N, K, tx.BF16, tx.F32, b_type=tx.F8E4M3,
                                scale_mode=tx.SCALE_MX32))
    assert plan.kernel == tx.KERNEL_GEMM_MX_BF16 and plan.workspace_bytes > 0
    c_ref = torch.empty((M, N), dtype=torch.float32, device=gpu)
    c_new = torch.full((M, N), float("nan"), dtype=torch.float32, device=gpu)
    ws = torch.empty(int(plan.workspace_bytes), dtype=torch.uint8, device=gpu)
    _launch("plain", plan, a, codes, c_ref, None, scales, ws)
    _launch("noalloc", plan, a, codes, c_new, None, scales)
    torch.cuda.synchronize()
    assert torch.equal(c_new.view(torch.int32), c_ref.view(torch.int32))


def test_noalloc_mx_upcast_then_decode(gpu):
    """The upcast writes after the counter region: a decode call after it still sees its
    counters at zero."""
    _mx_bf16(gpu, 512, 1024, 2048, 31)
    _mx_bf16(gpu, 256, 256, 512, 32)
    _w8a8(gpu, 16, 8192, 8192, 33)


def _decode16(gpu, M, N, K, seed):
    import torch
    say(f"noalloc bf16 decode M={M} N={N} K={K} seed={seed}")
    g = torch.Generator(device=gpu)
    g.manual_seed(seed)
    a = (torch.randn((M, K), generator=g, device=gpu) / K ** 0.5).to(torch.bfloat16)
    b = (torch.randn((K, N), generator=g, device=gpu) / K ** 0.5).to(torch.bfloat16)
    plan = tx.plan(tx.make_desc(M, N, K, tx.BF16, tx.F32))
    assert plan.kernel == tx.KERNEL_DECODE_16BIT and plan.workspace_bytes > 0
    c_ref = torch.empty((M, N), dtype=torch.float32, device=gpu)
    c_new = torch.full((M, N), float("nan"), dtype=torch.float32, device=gpu)
    ws = torch.zeros(int(plan.workspace_bytes), dtype=torch.uint8, device=gpu)
    _launch("plain", plan, a, b, c_ref, None, None, ws)
    _launch("noalloc", plan, a, b, c_new, None, None)
    torch.cuda.synchronize()
    assert torch.equal(c_new.view(torch.int32), c_ref.view(torch.int32))
    return plan


def test_noalloc_decode16_between_w8a8_calls(gpu):
    """The 16-bit decode kernel's fp32 partials and per-strip counters on the same scratch as
    the W8A8 decode: two decode16 calls (the second smaller), each after a W8A8 call, and a
    W8A8 call after them, all bit-equal to tx_dot_launch on a fresh workspace."""
    _w8a8(gpu, 16, 8192, 8192, 61)
    p1 = _decode16(gpu, 16, 8192, 8192, 62)
    _w8a8(gpu, 5, 2048, 4096, 63)
    p2 = _decode16(gpu, 3, 1024, 2048, 64)
    assert p1.split_k > 1 and p2.split_k > 1 and p2.workspace_bytes < p1.workspace_bytes
    _w8a8(gpu, 16, 8192, 8192, 65)


def test_noalloc_decode_f8(gpu):
    """The fp8 decode kernel (block-scaled, split-K) on the shared scratch, between W8A8
    calls, bit-equal to tx_dot_launch on a fresh workspace."""
    import torch
    from dotcase import fp8_block_inputs
    _w8a8(gpu, 16, 8192, 8192, 71)
    for M, N, K, seed in ((16, 7168, 7168, 72), (4, 1024, 2048, 73)):
        say(f"noalloc fp8 decode M={M} N={N} K={K}")
        qa, qb, sa, sb = fp8_block_inputs(M, N, K, seed)
        da, db, dsa, dsb = (to_device(x, gpu) for x in (qa, qb, sa, sb))
        plan = tx.plan(tx.make_desc(M, N, K, tx.F8E4M3, tx.BF16, scale_mode=tx.SCALE_BLOCK128))
        assert plan.kernel == tx.KERNEL_DECODE_F8 and plan.split_k > 1
        c_ref = torch.empty((M, N), dtype=torch.bfloat16, device=gpu)
        c_new = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu)
        ws = torch.zeros(int(plan.workspace_bytes), dtype=torch.uint8, device=gpu)
        _launch("plain", plan, da, db, c_ref, dsa, dsb, ws)
        _launch("noalloc", plan, da, db, c_new, dsa, dsb)
        torch.cuda.synchronize()
        assert torch.equal(c_new.view(torch.int16), c_ref.view(torch.int16))
    _w8a8(gpu, 16, 8192, 8192, 74)


def test_noalloc_kmajor_w8a8(gpu):
    """W8A8 with the weight kept [N][K] (B K-major) on the shared scratch: the 8-bit decode
    kernel's int8 form (M = 16) and the row kernel's K-major form (M = 100), larger call
    first, bit-equal to tx_dot_launch on a fresh workspace and to the oracle."""
    import torch
    for M, N, K, seed in ((100, 8192, 8192, 81), (16, 4096, 4096, 82), (16, 1000, 3000, 83)):
        say(f"noalloc W8A8 K-major M={M} N={N} K={K}")
        a, b = uniform_i8((M, K), seed), uniform_i8((K, N), seed + 1)
        sa, sb = uniform_scales(M, seed + 2), uniform_scales(N, seed + 3)
        lda = -(-K // 16) * 16
        pa = np.zeros((M, lda), dtype=np.int8)
        pa[:, :K] = a
        pbt = np.zeros((N, lda), dtype=np.int8)
        pbt[:, :K] = b.T
        da, dbt, dsa, dsb = (to_device(x, gpu) for x in (pa, pbt, sa, sb))
        plan = tx.plan(tx.make_desc(M, N, K, tx.I8, tx.BF16, scale_mode=tx.SCALE_ROWCOL,
                                    lda=lda, ldb=lda, ldc=-(-N // 8) * 8,
                                    flags=tx.FLAG_B_KMAJOR))
        assert plan.kernel == (tx.KERNEL_DECODE_I8 if M > 48 else tx.KERNEL_DECODE_F8)
        assert plan.split_k > 1
        ldc = plan.desc.ldc
        c_ref = torch.empty((M, ldc), dtype=torch.bfloat16, device=gpu)
        c_new = torch.full((M, ldc), float("nan"), dtype=torch.bfloat16, device=gpu)
        ws = torch.zeros(int(plan.workspace_bytes), dtype=torch.uint8, device=gpu)
        _launch("plain", plan, da, dbt, c_ref, dsa, dsb, ws)
        _launch("noalloc", plan, da, dbt, c_new, dsa, dsb)
        torch.cuda.synchronize()
        ref, got = from_device(c_ref)[:, :N], from_device(c_new)[:, :N]
        assert np.array_equal(got, ref), f"{np.count_nonzero(got != ref)} elements differ"
        orc = oracle.tiled_dot(a, b, a_type=oracle.I8, c_type=oracle.BF16, block=(64, 256, 128),
                               scale_mode=oracle.SCALE_ROWCOL, sa=sa, sb=sb)
        assert np.array_equal(got, orc)


def test_noalloc_split_k_tiles(gpu):
    """Split-K on the 256x256 tiles through the shared scratch: partials that fit run split
    (bit-equal to tx_dot_launch with a workspace); partials beyond the scratch (bf16
    M = 256, N = K = 8192: 64 MiB) run unsplit, within fp32 summation error of the exact
    product.  Then a W8A8 decode call on the same scratch."""
    import torch
    from dotcase import k_norm, normal_bf16
    for M, N, K, fits in ((200, 1000, 4096, True), (256, 8192, 8192, False)):
        say(f"noalloc split-K bf16 M={M} N={N} K={K}")
        a, b = normal_bf16((M, K), k_norm(K), M), normal_bf16((K, N), k_norm(K), N)
        da, db = to_device(a, gpu).view(torch.bfloat16), to_device(b, gpu).view(torch.bfloat16)
        plan = tx.plan(tx.make_desc(M, N, K, tx.BF16, tx.F32, ldc=-(-N // 4) * 4))
        assert plan.kernel == tx.KERNEL_GEMM_16BIT and plan.split_k > 1
        assert (plan.workspace_bytes <= tx.NOALLOC_SCRATCH_BYTES) == fits
        ldc = plan.desc.ldc
        c_ref = torch.empty((M, ldc), dtype=torch.float32, device=gpu)
        c_new = torch.full((M, ldc), float("nan"), dtype=torch.float32, device=gpu)
        ws = torch.empty(int(plan.workspace_bytes), dtype=torch.uint8, device=gpu)
        ws[:65536].zero_()
        _launch("plain", plan, da, db, c_ref, None, None, ws)
        _launch("noalloc", plan, da, db, c_new, None, None)
        torch.cuda.synchronize()
        ref, got = from_device(c_ref)[:, :N], from_device(c_new)[:, :N]
        if fits:
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
        exact = oracle.bf16_to_f32(a).astype(np.float64) @ oracle.bf16_to_f32(b).astype(np.float64)
        assert np.abs(got - exact).max() < 1e-5
    _w8a8(gpu, 16, 4096, 4096, 91)


def test_noalloc_workspace_free_kernels(gpu):
    """A plan without workspace (the bf16 tile) runs through the same entry point."""
    import torch
    say("noalloc bf16 300x264x200")
    g = torch.Generator(device=gpu)
    g.manual_seed(41)
    a = torch.randn((300, 200), generator=g, device=gpu).to(torch.bfloat16)
    b = torch.randn((200, 264), generator=g, device=gpu).to(torch.bfloat16)
    plan = tx.plan(tx.make_desc(300, 264, 200, tx.BF16, tx.F32))
    assert plan.workspace_bytes == 0
    c_ref = torch.empty((300, 264), dtype=torch.float32, device=gpu)
    c_new = torch.empty_like(c_ref)
    _launch("plain", plan, a, b, c_ref, None, None)
    _launch("noalloc", plan, a, b, c_new, None, None)
    torch.cuda.synchronize()
    assert torch.equal(c_new, c_ref)
