"""The 16-bit decode kernel (decode16.h) against the oracle.

bf16 / fp16 dots with M <= 96 stream B once on the decode kernel: strips of
64 columns (128 for slices of 32 .. 80 rows), 128-row K batches, split-K with the fp32 partials summed in split
order.  Parity is the north_star's fp bar: |d| <= 1e-3 + 1e-2 |ref| for inputs
N(0,1)/sqrt(K), against the oracle at the plan's block; fp32 C is also held to
the exact (float64) product within fp32 summation error.  Sums of fp32
partials depend on order, so the kernel fixes it: two launches give the same
bits.
"""
import numpy as np
import pytest

import oracle
import triton_ext_amd as tx
from dotcase import bits_to_f32, check_close, from_device, k_norm, normal_bf16, normal_f16, say, \
    to_device
from test_dot_gpu import ATOL, RTOL, oracle_16bit

pytestmark = pytest.mark.gpu

TORCH_DT = {"bf16": "bfloat16", "f16": "float16", "f32": "float32"}


def operands(M, N, K, kind, seed):
    gen = normal_bf16 if kind == "bf16" else normal_f16
    return gen((M, K), k_norm(K), 10 + seed), gen((K, N), k_norm(K), 20 + seed)


def run(gpu, a, b, kind, out_kind, acc=None):
    import torch
    tdt = getattr(torch, TORCH_DT[kind])
    da, db = to_device(a, gpu).view(tdt), to_device(b, gpu).view(tdt)
    c = tx.dot(da, db, out_dtype=getattr(torch, TORCH_DT[out_kind]),
               acc=None if acc is None else to_device(acc, gpu))
    torch.cuda.synchronize()
    return from_device(c)


def as_f32(x, kind):
    return x if kind == "f32" else bits_to_f32(x, kind)


def plan_of(M, N, K, kind, out_kind, flags=0):
    t = tx.BF16 if kind == "bf16" else tx.F16
    c = {"bf16": tx.BF16, "f16": tx.F16, "f32": tx.F32}[out_kind]
    up = lambda x: -(-x // 8) * 8
    return tx.plan(tx.make_desc(M, N, K, t, c, lda=up(K), ldb=up(N), ldc=up(N), flags=flags))


def exact(a, b, kind):
    f = oracle.bf16_to_f32 if kind == "bf16" else oracle.f16_to_f32
    return f(a).astype(np.float64) @ f(b).astype(np.float64)


@pytest.mark.parametrize("M,N,K,kind,out_kind", [
    (1, 8192, 8192, "bf16", "bf16"), (16, 8192, 8192, "bf16", "f32"),
    (64, 4096, 4096, "f16", "f16"), (48, 2048, 8192, "bf16", "bf16"),
    (16, 28672, 1024, "bf16", "bf16"), (8, 16384, 4096, "f16", "f32"),
    # ragged: K and N that fill no 16-byte chunk, slices of 16 .. 64 rows, one split
    (33, 4100, 2050, "bf16", "bf16"), (7, 1000, 3000, "f16", "f32"), (3, 24, 64, "bf16", "f32"),
    (64, 61, 300, "f16", "f16"), (17, 130, 129, "bf16", "f32"), (50, 520, 127, "f16", "f32"),
    # slices of 80 and 96 rows
    (80, 8192, 8192, "bf16", "bf16"), (96, 4096, 4096, "f16", "f32"),
    (90, 1000, 3000, "bf16", "f32"), (70, 61, 300, "f16", "f16"),
])
def test_decode16_vs_oracle(gpu, M, N, K, kind, out_kind):
    say(f"decode16 {kind}->{out_kind} M={M} N={N} K={K}")
    p = plan_of(M, N, K, kind, out_kind)
    assert p.kernel == tx.KERNEL_DECODE_16BIT
    a, b = operands(M, N, K, kind, M + K)
    got = as_f32(run(gpu, a, b, kind, out_kind), out_kind)
    ref = as_f32(oracle_16bit(a, b, kind, out_kind, (p.desc.block_m, p.desc.block_n,
                                                       p.desc.block_k)), out_kind)
    err = check_close(got, ref, atol=ATOL, rtol=RTOL, what=f"decode16 {M}x{N}x{K}")
    if out_kind == "f32":  # fp32 summation error only: K products of |x| <~ 4/sqrt(K) each
        assert np.abs(got - exact(a, b, kind)).max() < 1e-5
    say(f"decode16 {M}x{N}x{K} split {p.split_k}: max|d|={err:.3g}")


def test_decode16_k_zero(gpu):
    """K = 0: C = 0 (no batch is loaded)."""
    import torch
    for kind, out_kind in (("bf16", "bf16"), ("f16", "f32")):
        tdt = getattr(torch, TORCH_DT[kind])
        a = torch.empty((5, 0), dtype=tdt, device=gpu)
        b = torch.empty((0, 304), dtype=tdt, device=gpu)
        c = tx.dot(a, b, out_dtype=getattr(torch, TORCH_DT[out_kind]))
        torch.cuda.synchronize()
        assert not from_device(c).any()


@pytest.mark.parametrize("M,N,K", [(16, 8192, 8192), (5, 777, 1000)])
def test_decode16_accumulate(gpu, M, N, K):
    """tl.dot(a, b, acc) with an fp32 acc: C = acc + A @ B."""
    say(f"decode16 acc M={M} N={N} K={K}")
    assert plan_of(M, N, K, "bf16", "f32", tx.FLAG_ACCUMULATE).kernel == tx.KERNEL_DECODE_16BIT
    a, b = operands(M, N, K, "bf16", 3)
    acc = np.random.default_rng(4).standard_normal((M, N)).astype(np.float32)
    got = run(gpu, a, b, "bf16", "f32", acc=acc)
    ref = exact(a, b, "bf16") + acc
    assert np.abs(got - ref).max() < 1e-5


def test_decode16_inf_nan_padding(gpu):
    """Operands in storage whose row padding (past K in A, past N in B) and extra rows of
    B hold Inf and NaN: the chunks that cross K or N are loaded whole, and the
    elements past K must be zeroed (Inf * 0 = NaN) while those past N are never stored."""
    import torch
    M, N, K = 20, 1001, 1003
    say(f"decode16 Inf/NaN padding M={M} N={N} K={K}")
    a, b = operands(M, N, K, "bf16", 7)
    inf_bits, nan_bits = 0x7F80, 0x7FC0
    A = np.full((M, K + 13), inf_bits, dtype=np.uint16)
    A[:, K + 1::2] = nan_bits
    A[:, :K] = a
    B = np.full((K + 3, N + 7), nan_bits, dtype=np.uint16)
    B[:K, :N] = b
    da = to_device(A, gpu).view(torch.bfloat16)
    db = to_device(B, gpu).view(torch.bfloat16)
    c = tx.dot(da[:, :K], db[:K, :N], out_dtype=torch.float32)
    torch.cuda.synchronize()
    got = from_device(c)
    assert np.isfinite(got).all()
    assert np.abs(got - exact(a, b, "bf16")).max() < 1e-5


def test_decode16_deterministic(gpu):
    """Split-K partials are summed in split order: the same bits on every launch."""
    import torch
    M, N, K = 16, 1024, 8192
    p = plan_of(M, N, K, "bf16", "f32")
    assert p.split_k == 16
    a, b = operands(M, N, K, "bf16", 9)
    da, db = to_device(a, gpu).view(torch.bfloat16), to_device(b, gpu).view(torch.bfloat16)
    outs = []
    for _ in range(4):
        c = tx.dot(da, db, out_dtype=torch.float32)
        torch.cuda.synchronize()
        outs.append(from_device(c))
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32))


def test_decode16_after_w8a8_on_one_workspace(gpu):
    """The decode kernels share the workspace's counter region (every launch leaves its
    counters at zero): W8A8 split-K, then decode16 split-K, twice, on one buffer through
    tx_dot_launch."""
    import torch
    from test_workspace_gpu import _launch, _w8a8_case
    stream = torch.cuda.current_stream().cuda_stream
    M, N, K = 16, 4096, 4096
    pd = tx.plan(tx.make_desc(M, N, K, tx.I8, tx.BF16, scale_mode=tx.SCALE_ROWCOL))
    p16 = tx.plan(tx.make_desc(M, N, K, tx.BF16, tx.F32))
    assert pd.kernel == tx.KERNEL_DECODE_I8 and p16.kernel == tx.KERNEL_DECODE_16BIT
    assert pd.split_k > 1 and p16.split_k > 1
    ws = torch.zeros(max(int(pd.workspace_bytes), int(p16.workspace_bytes)), dtype=torch.uint8,
                     device=gpu)
    a8, b8, sa, sb, want8 = _w8a8_case(M, N, K, 81)
    d8 = [to_device(x, gpu) for x in (a8, b8, sa, sb)]
    a, b = operands(M, N, K, "bf16", 5)
    da, db = to_device(a, gpu).view(torch.bfloat16), to_device(b, gpu).view(torch.bfloat16)
    want16 = exact(a, b, "bf16")
    for rep in range(2):
        say(f"shared workspace: W8A8 then decode16 {M}x{N}x{K} (rep {rep})")
        c8 = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu)
        _launch(pd, d8[0], d8[1], c8, d8[2], d8[3], ws, stream)
        c16 = torch.full((M, N), float("nan"), dtype=torch.float32, device=gpu)
        _launch(p16, da, db, c16, None, None, ws, stream)
        torch.cuda.synchronize()
        assert np.array_equal(from_device(c8), want8)
        assert np.abs(from_device(c16) - want16).max() < 1e-5
    assert not from_device(ws[:65536]).any()  # every arrival counter back at zero


@pytest.mark.parametrize("M,N,K,kind,out_kind", [
    (16, 8192, 8192, "bf16", "f32"), (1, 4096, 4096, "f16", "f16"), (64, 1024, 2048, "bf16", "bf16"),
    (33, 4100, 2050, "bf16", "bf16"), (7, 1000, 3000, "f16", "f32"), (17, 130, 129, "bf16", "f32"),
    (50, 520, 127, "f16", "f32"), (5, 61, 1, "bf16", "f32"), (96, 1024, 2048, "bf16", "bf16"),
    (75, 520, 127, "f16", "f32")])
def test_decode16_kmajor_b(gpu, M, N, K, kind, out_kind):
    """B K-major (q @ k.T at decode; a weight kept [N][K]): B stored [N][K'] whose columns
    past K and rows past N hold NaN (A's padding holds Inf), so the chunk that crosses K
    must be zeroed on both sides.  Against the oracle, and against the same dot with B
    row-major: bit for bit with one batch a split (each lane's fragment holds the same K
    indices), else within fp32 summation order (each strip starts at its own batch)."""
    import torch
    say(f"decode16 K-major B {kind}->{out_kind} M={M} N={N} K={K}")
    tdt = getattr(torch, TORCH_DT[kind])
    odt = getattr(torch, TORCH_DT[out_kind])
    a, b = operands(M, N, K, kind, 5 * M + K)
    up = lambda x: -(-x // 8) * 8 + 8
    A = np.full((M, up(K)), 0x7F80 if kind == "bf16" else 0x7C00, dtype=np.uint16)
    A[:, :K] = a
    Bt = np.full((N + 3, up(K)), 0x7FC0 if kind == "bf16" else 0x7E00, dtype=np.uint16)
    Bt[:N, :K] = b.T
    da = to_device(A, gpu).view(tdt)[:, :K]
    db = to_device(Bt, gpu).view(tdt)[:N, :K].t()
    c = tx.dot(da, db, out_dtype=odt)
    p = tx.plan_for(da, db, tx.tx_type(c), ldc=c.stride(0))
    assert p.kernel == tx.KERNEL_DECODE_16BIT and p.desc.flags & tx.FLAG_B_KMAJOR
    c_row = tx.dot(da, to_device(b, gpu).view(tdt), out_dtype=odt)
    torch.cuda.synchronize()
    got = from_device(c)
    if -(-K // 128) <= p.split_k:  # at most one batch a split: the row-major order
        assert np.array_equal(got.view(np.uint8), from_device(c_row).view(np.uint8))
    ref = as_f32(oracle_16bit(a, b, kind, out_kind, (p.desc.block_m, p.desc.block_n,
                                                       p.desc.block_k)), out_kind)
    check_close(as_f32(got, out_kind), ref, atol=ATOL, rtol=RTOL, what=f"decode16 K-major")
    if out_kind == "f32":
        assert np.abs(got - exact(a, b, kind)).max() < 1e-5


def test_decode16_kmajor_b_accumulate_deterministic(gpu):
    """K-major B with an fp32 acc and split-K 16: C = acc + A @ B, the same bits on every
    launch."""
    import torch
    M, N, K = 16, 1024, 8192
    say(f"decode16 K-major B acc M={M} N={N} K={K}")
    a, b = operands(M, N, K, "bf16", 11)
    da = to_device(a, gpu).view(torch.bfloat16)
    db = to_device(np.ascontiguousarray(b.T), gpu).view(torch.bfloat16).t()
    acc = np.random.default_rng(12).standard_normal((M, N)).astype(np.float32)
    dacc = to_device(acc, gpu)
    p = tx.plan_for(da, db, tx.F32, flags=tx.FLAG_ACCUMULATE)
    assert p.kernel == tx.KERNEL_DECODE_16BIT and p.split_k == 16
    outs = []
    for _ in range(3):
        c = tx.dot(da, db, acc=dacc)
        torch.cuda.synchronize()
        outs.append(from_device(c))
    assert np.abs(outs[0] - (exact(a, b, "bf16") + acc)).max() < 1e-5
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32))


@pytest.mark.parametrize("M,N,K,kind,out_kind,kmajor", [
    (70, 1000, 3000, "bf16", "f32", False), (70, 1000, 3000, "f16", "f16", True),
    (5, 136, 136, "bf16", "bf16", False), (33, 4104, 2056, "bf16", "f32", True),
    (80, 8192, 8192, "f16", "f32", False), (64, 56, 304, "bf16", "f32", True),
    (48, 200, 1000, "f16", "f32", False)])
def test_decode16_strip_widths(gpu, M, N, K, kind, out_kind, kmajor):
    """Strips of 64 and of 128 columns, named by explicit block, on ragged shapes (N past the
    strip, K past the batch, rows past M), B row-major or K-major: each against the oracle and,
    in fp32, against the exact product within fp32 summation error."""
    import torch
    say(f"decode16 strip widths {kind}->{out_kind} M={M} N={N} K={K} kmajor={kmajor}")
    tdt = getattr(torch, TORCH_DT[kind])
    odt = getattr(torch, TORCH_DT[out_kind])
    a, b = operands(M, N, K, kind, 3 * M + N)
    da = to_device(a, gpu).view(tdt)
    db = (to_device(np.ascontiguousarray(b.T), gpu).view(tdt).t() if kmajor
          else to_device(b, gpu).view(tdt))
    sr = 16 * -(-M // 16)
    for w in (64, 128):
        c = tx.dot(da, db, out_dtype=odt, block=(sr, w, 128))
        torch.cuda.synchronize()
        p = tx.plan_for(da, db, tx.tx_type(c), block=(sr, w, 128), ldc=c.stride(0))
        assert p.kernel == tx.KERNEL_DECODE_16BIT and p.desc.block_n == w
        assert p.grid_x == -(-N // w) * p.split_k
        got = from_device(c)
        ref = as_f32(oracle_16bit(a, b, kind, out_kind, (sr, w, 128)), out_kind)
        check_close(as_f32(got, out_kind), ref, atol=ATOL, rtol=RTOL,
                    what=f"decode16 W={w} {M}x{N}x{K}")
        if out_kind == "f32":
            assert np.abs(got - exact(a, b, kind)).max() < 1e-5
