"""GPU parity of the fused attention forward (tx_attn_fwd_launch) against the
CPU oracle and, as the tutorial's own test does, a torch reference.

Bars: o within 1e-2 absolute of the reference (the tutorial's test_op,
R:pass/LoopSplit/06-fused-attention.py:698-718) and, against the oracle,
within 2^-8 (two fp16 ulps at |o| ~ 1: p is rounded to fp16 on both sides,
exp2 and the summation orders differ); M (base-2 logsumexp) within 1e-4.
e5m2 (the tutorial's fp8 provider): see check_e5m2.
"""
import os

import numpy as np
import pytest

import oracle
import triton_ext_amd as tx
from dotcase import from_device, say, to_device

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def rand_qkv(Z, H, N, D, seed, std=0.5):
    rng = np.random.default_rng(seed)
    return [(rng.standard_normal((Z, H, N, D)) * std).astype(np.float16).view(np.uint16)
            for _ in range(3)]


def run_gpu(gpu, q, k, v, causal, sm_scale, layout="bhnd", block=(0, 0)):
    import torch
    ts = []
    for x in (q, k, v):
        t = to_device(x, gpu).view(torch.float16)
        if layout == "bnhd":  # storage [Z, N, H, D], viewed as [Z, H, N, D]
            t = t.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)
        ts.append(t)
    o, M = tx.attention(*ts, causal, sm_scale, return_lse=True, block=block)
    torch.cuda.synchronize()
    return from_device(o.contiguous().view(torch.int16)).view(np.uint16), from_device(M)


def check(o, M, ro, rM, what, tol=2.0 ** -8):
    go = o.view(np.float16).astype(np.float64)
    wo = ro.view(np.float16).astype(np.float64)
    assert np.isfinite(go).all(), f"{what}: non-finite o"
    d = np.abs(go - wo)
    assert d.max() <= tol, f"{what}: max |d o| {d.max():.3g} (bound {tol:.3g})"
    dm = np.abs(M.reshape(rM.shape).astype(np.float64) - rM)
    assert dm.max() <= 1e-4 * max(1.0, np.abs(rM).max()), f"{what}: max |d M| {dm.max():.3g}"
    say(f"{what}: max|d o|={d.max():.3g} identical={np.mean(go == wo):.3f} max|d M|={dm.max():.3g}")


def test_tutorial_test_op(gpu):
    """The tutorial's test_op: (1, 2, 1024, 64), causal, N(0, 0.5) fp16,
    sm_scale 0.5, against softmax in fp32 -> fp16 -> matmul, atol 1e-2."""
    import torch
    say("attn test_op (1, 2, 1024, 64) causal")
    q, k, v = rand_qkv(1, 2, 1024, 64, seed=20)
    o, _ = run_gpu(gpu, q, k, v, True, 0.5)
    qt, kt, vt = (torch.from_numpy(x.view(np.float16)).float() for x in (q, k, v))
    N = 1024
    Mk = torch.tril(torch.ones((N, N)))
    p = torch.matmul(qt, kt.transpose(2, 3)) * 0.5
    p[:, :, Mk == 0] = float("-inf")
    p = torch.softmax(p, dim=-1).half().float()
    ref = torch.matmul(p, vt).half()
    got = torch.from_numpy(o.view(np.float16))
    assert torch.allclose(ref, got, atol=1e-2, rtol=0)
    # the tutorial's positional USE_TMA: one tensor back, the same bits
    qd, kd, vd = (to_device(x, gpu).view(torch.float16) for x in (q, k, v))
    o2 = tx.attention(qd, kd, vd, True, 0.5, True)
    torch.cuda.synchronize()
    assert isinstance(o2, torch.Tensor)
    assert np.array_equal(from_device(o2.view(torch.int16)).view(np.uint16), o)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("Z,H,N,sm_scale,layout", [(1, 2, 256, 0.5, "bhnd"),
                                                   (2, 3, 384, 1.3, "bhnd"),
                                                   (1, 4, 512, 0.125, "bnhd"),
                                                   (1, 1, 128, 0.5, "bhnd")])
def test_attn_vs_oracle(gpu, causal, Z, H, N, sm_scale, layout):
    say(f"attn Z={Z} H={H} N={N} causal={causal} scale={sm_scale} {layout}")
    q, k, v = rand_qkv(Z, H, N, 64, seed=Z * 100 + H * 10 + N + causal)
    o, M = run_gpu(gpu, q, k, v, causal, sm_scale, layout)
    ro, rM = oracle.attn_fwd(q, k, v, sm_scale=sm_scale, causal=causal, block=(128, 64))
    check(o, M, ro, rM, f"attn {Z}x{H}x{N} causal={causal} {layout}")


@pytest.mark.parametrize("own_block", [False, True])
@pytest.mark.parametrize("name", ["attn_fwd_causal", "attn_fwd_plain"])
def test_golden_fixture_attn(gpu, name, own_block):
    """The interpreter's fixtures (written with BLOCK 64 x 32) on the default
    128 x 64 kernel and on the fixture's own block shape."""
    z = np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)
    block = tuple(int(x) for x in z["block"]) if own_block else (0, 0)
    say(f"golden {name} block={block}")
    o, M = run_gpu(gpu, z["q"], z["k"], z["v"], bool(z["causal"]), float(z["sm_scale"]),
                   block=block)
    check(o, M, z["o"], z["M"], f"golden {name} block={block}")


@pytest.mark.parametrize("block", [(128, 32), (64, 64), (64, 32)])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("Z,H,N,D,bf16", [(1, 2, 64, 64, False), (2, 3, 192, 64, False),
                                          (1, 2, 320, 128, False), (1, 2, 256, 64, True),
                                          (1, 1, 128, 128, True)])
def test_attn_blocks_vs_oracle(gpu, block, causal, Z, H, N, D, bf16):
    """The tutorial's other autotuned blocks (BLOCK_M 64 / 128 by BLOCK_N 32 /
    64) against the oracle run with the same blocks.  N_CTX = 64, 192, 320
    give odd block counts in both loop segments at BLOCK_M 64."""
    attn_vs_oracle(gpu, block, causal, Z, H, N, D, bf16)


@pytest.mark.parametrize("block", [(128, 64), (128, 32), (64, 64), (64, 32)])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("Z,H,N,D,bf16", [(2, 2, 256, 32, False), (1, 3, 192, 32, True),
                                          (1, 2, 256, 256, False), (2, 1, 192, 256, True),
                                          (2, 2, 256, 16, False), (1, 3, 192, 16, True)])
def test_attn_head_dims_16_32_and_256(gpu, block, causal, Z, H, N, D, bf16):
    """Head dims 32 and 256 (64- and 512-byte K/V rows, their own swizzles; 256 reads its
    fragments in groups), and 16 (staged as 32 with zero dims past 16, O's not stored), at
    every block shape; at 128 x 32, head dims 16 and 32 give a 2 KiB K block that waves
    0 and 1 load for all four."""
    attn_vs_oracle(gpu, block, causal, Z, H, N, D, bf16)


def attn_vs_oracle(gpu, block, causal, Z, H, N, D, bf16):
    """fp16 / bf16 attention at `block` against the oracle at the same block."""
    import torch
    if N % block[0]:
        pytest.skip("N_CTX is not a whole number of BLOCK_M blocks")
    say(f"attn block={block} Z={Z} H={H} N={N} D={D} bf16={bf16} causal={causal}")
    rng = np.random.default_rng(N * 3 + D + causal + bf16 + block[0] + block[1])
    tdt = torch.bfloat16 if bf16 else torch.float16
    bits = [torch.from_numpy((rng.standard_normal((Z, H, N, D)) * 0.5).astype(np.float32))
            .to(tdt).view(torch.int16).numpy().view(np.uint16) for _ in range(3)]
    ts = [to_device(b, gpu).view(torch.int16).view(tdt) for b in bits]
    o, M = tx.attention(*ts, causal, 0.6, return_lse=True, block=block)
    torch.cuda.synchronize()
    got = from_device(o.contiguous().view(torch.int16)).view(np.uint16)
    ro, rM = oracle.attn_fwd(*bits, sm_scale=0.6, causal=causal, block=block,
                             dtype=oracle.BF16 if bf16 else oracle.F16)
    dec = (lambda x: oracle.bf16_to_f32(x).astype(np.float64)) if bf16 else \
        (lambda x: x.view(np.float16).astype(np.float64))
    d = np.abs(dec(got) - dec(ro))
    tol = 2.0 ** -6 if bf16 else 2.0 ** -8
    assert np.isfinite(dec(got)).all()
    assert d.max() <= tol, f"max |d o| {d.max():.3g}"
    dm = np.abs(from_device(M).reshape(rM.shape).astype(np.float64) - rM)
    assert dm.max() <= 1e-4 * max(1.0, np.abs(rM).max()), f"max |d M| {dm.max():.3g}"
    say(f"attn block={block}: max|d o|={d.max():.3g} identical={np.mean(got == ro):.3f}")


@pytest.mark.parametrize("causal", [True, False])
def test_attn_bench_shape_sampled_heads(gpu, causal):
    """The bench shape (4, 32, 4096, 64): every program runs; two heads are
    checked in full against the oracle."""
    import torch
    say(f"attn 4x32x4096 causal={causal}")
    Z, H, N, D = 4, 32, 4096, 64
    g = torch.Generator(device=gpu)
    g.manual_seed(5)
    q, k, v = (torch.randn((Z, H, N, D), generator=g, device=gpu, dtype=torch.float16) * 0.5
               for _ in range(3))
    o, M = tx.attention(q, k, v, causal, 0.5, return_lse=True)
    torch.cuda.synchronize()
    assert torch.isfinite(o).all()
    for (zi, hi) in ((0, 0), (3, 31)):
        sub = [from_device(t[zi:zi + 1, hi:hi + 1].contiguous().view(torch.int16)).view(np.uint16)
               for t in (q, k, v)]
        ro, rM = oracle.attn_fwd(*sub, sm_scale=0.5, causal=causal, block=(128, 64))
        got = from_device(o[zi:zi + 1, hi:hi + 1].contiguous().view(torch.int16)).view(np.uint16)
        check(got, from_device(M[zi, hi]), ro, rM, f"attn 4x32x4096 head ({zi},{hi})")


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("D,bf16,Z,H,N,layout", [(128, False, 2, 3, 384, "bhnd"),
                                                 (64, True, 2, 3, 384, "bhnd"),
                                                 (128, True, 1, 2, 1024, "bnhd")])
def test_attn_head_dim_128_and_bf16(gpu, causal, D, bf16, Z, H, N, layout):
    """Head dim 128 (256-byte K/V rows, their own swizzles) and bf16 (p and
    o rounded to nearest even) against the oracle."""
    import torch
    say(f"attn D={D} bf16={bf16} Z={Z} H={H} N={N} causal={causal} {layout}")
    rng = np.random.default_rng(D * 7 + N + causal + bf16)
    tdt = torch.bfloat16 if bf16 else torch.float16
    bits = [torch.from_numpy((rng.standard_normal((Z, H, N, D)) * 0.5).astype(np.float32))
            .to(tdt).view(torch.int16).numpy().view(np.uint16) for _ in range(3)]
    ts = []
    for b in bits:
        t = to_device(b, gpu).view(torch.int16).view(tdt)
        if layout == "bnhd":
            t = t.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)
        ts.append(t)
    o, M = tx.attention(*ts, causal, 0.7, return_lse=True)
    torch.cuda.synchronize()
    got = from_device(o.contiguous().view(torch.int16)).view(np.uint16)
    ro, rM = oracle.attn_fwd(*bits, sm_scale=0.7, causal=causal, block=(128, 64),
                             dtype=oracle.BF16 if bf16 else oracle.F16)
    dec = lambda b: torch.from_numpy(b.view(np.int16)).view(tdt).double().numpy()
    d = np.abs(dec(got) - dec(ro))
    tol = 2.0 ** -6 if bf16 else 2.0 ** -8
    assert np.isfinite(dec(got)).all()
    assert d.max() <= tol, f"max |d o| {d.max():.3g}"
    dm = np.abs(from_device(M).reshape(rM.shape).astype(np.float64) - rM)
    assert dm.max() <= 1e-4 * max(1.0, np.abs(rM).max()), f"max |d M| {dm.max():.3g}"
    say(f"attn D={D} bf16={bf16}: max|d o|={d.max():.3g} identical={np.mean(got == ro):.3f}")


# --- fp8 e5m2 (the tutorial's fp8 provider) ---------------------------------

def e5m2_qkv(Z, H, N, D, seed, std=1.0):
    """The tutorial's fp8 bench inputs: randn fp16, then .to(float8_e5m2)."""
    import torch
    rng = np.random.default_rng(seed)
    return [torch.from_numpy((rng.standard_normal((Z, H, N, D)) * std).astype(np.float16))
            .to(torch.float8_e5m2).view(torch.uint8).numpy() for _ in range(3)]


def run_gpu_fp8(gpu, q, k, v, causal, sm_scale, block=(0, 0)):
    """q, k head-dim contiguous; v stored key-contiguous and viewed as
    [Z, H, N, D], as the tutorial's v.permute(0, 1, 3, 2).contiguous()
    .permute(0, 1, 3, 2) leaves it."""
    import torch
    qt, kt = (to_device(x, gpu).view(torch.float8_e5m2) for x in (q, k))
    vt = to_device(np.ascontiguousarray(v.transpose(0, 1, 3, 2)), gpu).view(torch.float8_e5m2)
    vt = vt.permute(0, 1, 3, 2)
    assert vt.stride(2) == 1
    o, M = tx.attention(qt, kt, vt, causal, sm_scale, return_lse=True, block=block)
    torch.cuda.synchronize()
    assert o.dtype == torch.float8_e5m2
    return o.view(torch.uint8).cpu().numpy(), from_device(M)


def e5m2_step(x):
    """Spacing of e5m2 values at |x| (2^-16 in the subnormal range)."""
    a = np.maximum(np.abs(x), 2.0 ** -14)
    return 2.0 ** (np.floor(np.log2(a)) - 2)


def check_e5m2(o, M, ro, rM, codes, sm_scale, causal, what):
    """Parity of e5m2 outputs.  p and o are rounded to nearest even on both
    sides; their fp32 values differ slightly (summation order, the MFMA's
    group sums, v_exp_f32), so a value lying at a rounding boundary can land
    on either side.  An o code then moves one step, and a p code moves one
    step, changing o by at most 2^-2 p_n |v_n| / l.  The bar: every
    difference within one e5m2 step of o plus one p flip of the row's largest
    term, 2^-2 max_n p_n |v_n| / l (float64 softmax of the decoded inputs),
    and at least 99% of o codes identical, less one row of D codes: a single
    p flip moves o in every column of its row, which on a one-head 64-row
    output is 1.6% of the codes at D = 32."""
    import torch
    dec = lambda c: torch.from_numpy(np.ascontiguousarray(c)).view(torch.float8_e5m2) \
        .double().numpy()
    a, b = dec(o), dec(ro)
    qf, kf, vf = (dec(c) for c in codes)
    N = qf.shape[2]
    s = np.einsum("zhmd,zhnd->zhmn", qf, kf) * sm_scale
    if causal:
        s = np.where(np.tril(np.ones((N, N))) > 0, s, -np.inf)
    P = np.exp(s - s.max(-1, keepdims=True))
    P /= P.sum(-1, keepdims=True)
    top = np.empty(a.shape)  # max_n p_n |v_n| / l, [Z, H, M, D], in row chunks
    for r in range(0, N, 64):
        top[:, :, r:r + 64] = np.max(P[:, :, r:r + 64, :, None] * np.abs(vf)[:, :, None],
                                     axis=-2)
    assert ((o & 0x7F) < 0x7C).all(), f"{what}: inf/NaN in o"
    same = np.mean(o == ro)
    assert same >= 0.99 - o.shape[-1] / o.size, f"{what}: only {same:.4f} of o codes identical"
    excess = np.abs(a - b) - (e5m2_step(np.maximum(np.abs(a), np.abs(b))) + top / 4)
    assert excess.max() <= 0, f"{what}: |d o| exceeds its bound by {excess.max():.3g} " \
        f"(identical {same:.4f})"
    dm = np.abs(M.reshape(rM.shape).astype(np.float64) - rM)
    assert dm.max() <= 1e-4 * max(1.0, np.abs(rM).max()), f"{what}: max |d M| {dm.max():.3g}"
    say(f"{what}: identical={same:.4f} max|d o|={np.abs(a - b).max():.3g} max|d M|={dm.max():.3g}")


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("Z,H,N,D,sm_scale", [(1, 2, 256, 64, 1.3), (2, 3, 384, 64, 0.5),
                                              (1, 1, 128, 64, 0.3), (1, 2, 512, 128, 0.3),
                                              (2, 1, 256, 128, 1.3)])
def test_attn_fp8_vs_oracle(gpu, causal, Z, H, N, D, sm_scale):
    say(f"attn fp8 Z={Z} H={H} N={N} D={D} causal={causal} scale={sm_scale}")
    q, k, v = e5m2_qkv(Z, H, N, D, seed=Z * 100 + H * 10 + N + D + causal)
    o, M = run_gpu_fp8(gpu, q, k, v, causal, sm_scale)
    ro, rM = oracle.attn_fwd(q, k, v, sm_scale=sm_scale, causal=causal, block=(128, 64),
                             dtype=oracle.F8E5M2)
    check_e5m2(o, M, ro, rM, (q, k, v), sm_scale, causal,
               f"attn fp8 {Z}x{H}x{N} D={D} causal={causal}")


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("Z,H,N,D", [(1, 2, 64, 64), (2, 3, 192, 64), (1, 2, 320, 128)])
def test_attn_fp8_block_m64(gpu, causal, Z, H, N, D):
    """fp8 e5m2 with BLOCK_M 64 (two waves), against the oracle at 64 x 64."""
    say(f"attn fp8 block=(64, 64) Z={Z} H={H} N={N} D={D} causal={causal}")
    q, k, v = e5m2_qkv(Z, H, N, D, seed=Z * 100 + H * 10 + N + D + causal + 7)
    o, M = run_gpu_fp8(gpu, q, k, v, causal, 0.7, block=(64, 64))
    ro, rM = oracle.attn_fwd(q, k, v, sm_scale=0.7, causal=causal, block=(64, 64),
                             dtype=oracle.F8E5M2)
    check_e5m2(o, M, ro, rM, (q, k, v), 0.7, causal,
               f"attn fp8 block 64x64 {Z}x{H}x{N} D={D} causal={causal}")


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("Z,H,N,D,block", [(1, 2, 256, 16, (128, 64)), (2, 1, 192, 16, (64, 64)),
                                           (1, 2, 384, 32, (128, 64)), (1, 3, 128, 32, (64, 64)),
                                           (1, 2, 256, 256, (128, 64)),
                                           (2, 1, 192, 256, (64, 64))])
def test_attn_fp8_head_dims_16_32_and_256(gpu, causal, Z, H, N, D, block):
    """The tutorial's other fp8 head dims: 16 and 32 run in the layout of 64
    (K chunks and V^T rows past the head dim read as zeros), 256 in 256-byte
    K rows."""
    say(f"attn fp8 D={D} block={block} Z={Z} H={H} N={N} causal={causal}")
    q, k, v = e5m2_qkv(Z, H, N, D, seed=Z * 100 + H * 10 + N + D + causal + 11)
    o, M = run_gpu_fp8(gpu, q, k, v, causal, 0.6, block=block)
    ro, rM = oracle.attn_fwd(q, k, v, sm_scale=0.6, causal=causal, block=block,
                             dtype=oracle.F8E5M2)
    check_e5m2(o, M, ro, rM, (q, k, v), 0.6, causal,
               f"attn fp8 D={D} block={block} {Z}x{H}x{N} causal={causal}")


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("Z,H,N,D,block", [(1, 2, 64, 64, (64, 32)), (2, 3, 192, 64, (64, 32)),
                                           (1, 2, 256, 16, (64, 32)), (1, 3, 192, 32, (64, 32)),
                                           (1, 2, 320, 128, (64, 32)), (2, 1, 256, 128, (128, 32)),
                                           (1, 2, 384, 256, (128, 32)), (2, 1, 192, 256, (64, 32)),
                                           (1, 2, 256, 16, (128, 32)), (2, 1, 384, 32, (128, 32)),
                                           (1, 3, 256, 64, (128, 32))])
def test_attn_fp8_block_n32(gpu, causal, Z, H, N, D, block):
    """fp8 e5m2 with BLOCK_N 32: one 32-key block per S^T MFMA and half of
    each P V MFMA (the other half of P and V^T zero bytes in registers),
    against the oracle at the same blocks.  N_CTX = 64, 192, 320 give odd
    block counts at BLOCK_M 64; head dims 16 and 32 run in the layout of 64, and
    with 64 at 128 x 32 their 2 KiB K and V^T blocks are loaded by two of the
    four waves."""
    say(f"attn fp8 block={block} Z={Z} H={H} N={N} D={D} causal={causal}")
    q, k, v = e5m2_qkv(Z, H, N, D, seed=Z * 100 + H * 10 + N + D + causal + 13)
    o, M = run_gpu_fp8(gpu, q, k, v, causal, 0.8, block=block)
    ro, rM = oracle.attn_fwd(q, k, v, sm_scale=0.8, causal=causal, block=block,
                             dtype=oracle.F8E5M2)
    check_e5m2(o, M, ro, rM, (q, k, v), 0.8, causal,
               f"attn fp8 block={block} {Z}x{H}x{N} D={D} causal={causal}")


@pytest.mark.parametrize("causal", [True, False])
def test_attn_fp8_bench_shape_sampled_heads(gpu, causal):
    """The tutorial's fp8 bench shape (4, 32, 4096, 64), sm_scale 1.3: every
    program runs; two heads are checked in full against the oracle."""
    import torch
    say(f"attn fp8 4x32x4096 causal={causal}")
    Z, H, N, D = 4, 32, 4096, 64
    g = torch.Generator(device=gpu)
    g.manual_seed(6)
    q, k, v = (torch.randn((Z, H, N, D), generator=g, device=gpu, dtype=torch.float16)
               .to(torch.float8_e5m2) for _ in range(3))
    vt = v.permute(0, 1, 3, 2).contiguous().permute(0, 1, 3, 2)
    o, M = tx.attention(q, k, vt, causal, 1.3, return_lse=True)
    torch.cuda.synchronize()
    assert ((o.view(torch.uint8) & 0x7F) < 0x7C).all()
    for (zi, hi) in ((0, 0), (3, 31)):
        sub = [t[zi:zi + 1, hi:hi + 1].contiguous().view(torch.uint8).cpu().numpy()
               for t in (q, k, v)]
        ro, rM = oracle.attn_fwd(*sub, sm_scale=1.3, causal=causal, block=(128, 64),
                                 dtype=oracle.F8E5M2)
        got = o[zi:zi + 1, hi:hi + 1].contiguous().view(torch.uint8).cpu().numpy()
        check_e5m2(got, from_device(M[zi, hi]), ro, rM, sub, 1.3, causal,
                   f"attn fp8 4x32x4096 head ({zi},{hi})")
