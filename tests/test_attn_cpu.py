"""Fused attention forward: the CPU oracle's pins and the C-ABI plan checks.

oracle_attn_fwd (oracle/tiled_dot.c) restates the forward of the reference's
fused-attention tutorial (R:pass/LoopSplit/06-fused-attention.py:44-93,
:181-239).  Pinned by:
  1. golden fixtures of the Triton interpreter running that forward
     (tests/golden/attn_*.npz, make_golden.py's attn_fwd_kernel);
  2. mathematics: exact float64 softmax(q k^T sm_scale [+ causal mask]) v and
     the base-2 logsumexp M, within fp16 / fp32 rounding;
  3. the LoopSplit claim the tutorial relies on: the split loop (off-band
     unmasked, on-band masked) equals the loop with every block masked, bit
     for bit, and so does skipping the blocks past the diagonal (what the GPU
     kernel does).
The fp8 provider (e5m2 q, k, v, p and o) adds two codecs for p.to(fp8e5) and
o.to(fp8e5): round to nearest even (compiled Triton, the GPU kernel), pinned
against torch's float8_e5m2 cast, and the interpreter's own converter, pinned
bit for bit against the interpreter's cast (tests/golden/e5m2_cast_interp.npz);
the attention fixtures attn_fwd_fp8_* pin the forward with the latter.
"""
import glob
import os

import numpy as np
import pytest

import oracle
import triton_ext_amd as tx

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def rand_qkv(Z, H, N, D, seed, std=0.5):
    rng = np.random.default_rng(seed)
    return [(rng.standard_normal((Z, H, N, D)) * std).astype(np.float16).view(np.uint16)
            for _ in range(3)]


def exact_attention(q, k, v, sm_scale, causal):
    """float64: o = softmax(q k^T sm_scale) v and M = log2 sum_n 2^(qk_scale qk)."""
    qf, kf, vf = (x.view(np.float16).astype(np.float64) for x in (q, k, v))
    N = q.shape[2]
    s = np.einsum("zhmd,zhnd->zhmn", qf, kf)
    qk_scale = float(np.float32(sm_scale) * np.float32(1.44269504))
    if causal:
        s = np.where(np.tril(np.ones((N, N))) > 0, s, -np.inf)
    t = s * qk_scale
    mx = t.max(-1, keepdims=True)
    p = np.exp2(t - mx)
    lse = (mx[..., 0] + np.log2(p.sum(-1)))
    o = (p / p.sum(-1, keepdims=True)) @ vf
    return o, lse.reshape(-1, N)


ATTN_FIXTURES = sorted(p for p in glob.glob(os.path.join(GOLDEN, "attn_*.npz"))
                       if "_fp8_" not in p)
FP8_FIXTURES = sorted(glob.glob(os.path.join(GOLDEN, "attn_fwd_fp8_*.npz")))


def e5m2_values(codes):
    import torch
    return torch.from_numpy(np.ascontiguousarray(codes)).view(torch.float8_e5m2).double().numpy()


@pytest.mark.parametrize("path", ATTN_FIXTURES,
                         ids=[os.path.basename(p)[:-4] for p in ATTN_FIXTURES])
def test_golden_fixture_attn(path):
    z = np.load(path, allow_pickle=False)
    o, M = oracle.attn_fwd(z["q"], z["k"], z["v"], sm_scale=float(z["sm_scale"]),
                           causal=bool(z["causal"]), block=tuple(int(x) for x in z["block"]))
    go = o.view(np.float16).astype(np.float32)
    wo = z["o"].view(np.float16).astype(np.float32)
    # same steps, different fp32 summation order (np.matmul / np.sum): at most
    # an fp16 ulp of |o| <= 2 apart
    assert np.abs(go - wo).max() <= 2 ** -9, np.abs(go - wo).max()
    assert np.mean(go == wo) > 0.98
    assert np.abs(M - z["M"]).max() <= 1e-5 * np.abs(z["M"]).max() + 1e-6


def test_e5m2_codecs():
    """p.to(fp8e5) and o.to(fp8e5): RNE against torch over a wide sweep, the
    interpreter's converter against the interpreter's own cast bit for bit."""
    import torch
    z = np.load(os.path.join(GOLDEN, "e5m2_cast_interp.npz"), allow_pickle=False)
    x, y = z["x"], z["y"]
    assert np.array_equal(oracle.f32_to_e5m2(x, oracle.ROUND_INTERP), y)
    rng = np.random.default_rng(7)
    sweep = np.concatenate([x, np.concatenate(
        [rng.standard_normal(50000).astype(np.float32) * np.float32(s)
         for s in (1e-6, 1e-4, 1e-2, 1.0, 1e2, 1e4)]),
        np.arange(-70000, 70000, 0.37, dtype=np.float32)])
    want = torch.from_numpy(sweep).to(torch.float8_e5m2).view(torch.uint8).numpy()
    assert np.array_equal(oracle.f32_to_e5m2(sweep, oracle.ROUND_RNE), want)
    # the two differ (half-up vs half-even, the carry ORed into the exponent):
    # 0.4921875 = 1.96875 * 2^-2 is 0.5 to nearest and 0.25 in the interpreter
    v = np.array([0.4921875, 0.375 + 2 ** -5], np.float32)
    assert list(e5m2_values(oracle.f32_to_e5m2(v))) == [0.5, 0.375]
    assert list(e5m2_values(oracle.f32_to_e5m2(v, oracle.ROUND_INTERP))) == [0.25, 0.4375]


@pytest.mark.parametrize("path", FP8_FIXTURES, ids=[os.path.basename(p)[:-4] for p in FP8_FIXTURES])
def test_golden_fixture_attn_fp8(path):
    """The interpreter running the tutorial's fp8 forward (e5m2 q, k, v, p,
    o) against the oracle with the interpreter's converter: o codes agree but
    where a different fp32 summation order lands on the other side of a
    rounding boundary (there the converter's carry quirk can halve a value)."""
    z = np.load(path, allow_pickle=False)
    o, M = oracle.attn_fwd(z["q"], z["k"], z["v"], sm_scale=float(z["sm_scale"]),
                           causal=bool(z["causal"]), block=tuple(int(x) for x in z["block"]),
                           dtype=oracle.F8E5M2, round_mode=oracle.ROUND_INTERP)
    assert np.mean(o == z["o"]) > 0.99
    a, b = e5m2_values(o), e5m2_values(z["o"])
    m = a != b
    assert (np.abs(a[m] - b[m]) <= 0.5 * np.maximum(np.abs(a[m]), np.abs(b[m])) + 2 ** -16).all()
    assert np.abs(M - z["M"]).max() <= 1e-5 * np.abs(z["M"]).max() + 1e-6
    # and with round to nearest even (the GPU kernel's rounding) the same
    # forward moves a share of the codes
    o_rne, M_rne = oracle.attn_fwd(z["q"], z["k"], z["v"], sm_scale=float(z["sm_scale"]),
                                   causal=bool(z["causal"]),
                                   block=tuple(int(x) for x in z["block"]), dtype=oracle.F8E5M2)
    assert 0.5 < np.mean(o_rne == z["o"]) < 0.99


@pytest.mark.parametrize("causal", [True, False])
def test_attn_oracle_fp8_vs_float64(causal):
    """e5m2 forward (round to nearest even) against float64 attention of the
    same decoded inputs: p and o each carry e5m2's 2^-3 relative rounding."""
    import torch
    rng = np.random.default_rng(11 + causal)
    codes = [torch.from_numpy(rng.standard_normal((1, 2, 256, 64)).astype(np.float16))
             .to(torch.float8_e5m2).view(torch.uint8).numpy() for _ in range(3)]
    qf, kf, vf = (e5m2_values(c) for c in codes)
    o, M = oracle.attn_fwd(*codes, sm_scale=0.3, causal=causal, block=(128, 64),
                           dtype=oracle.F8E5M2)
    N = 256
    s = np.einsum("zhmd,zhnd->zhmn", qf, kf) * 0.3
    if causal:
        s = np.where(np.tril(np.ones((N, N))) > 0, s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    ref = (p / p.sum(-1, keepdims=True)) @ vf
    got = e5m2_values(o)
    # |sum p eps v| / l <= 2^-3 max|v| per row, then o's own rounding
    bound = 2 ** -3 * np.abs(vf).max(axis=(2, 3), keepdims=True) + 2 ** -3 * np.abs(ref)
    assert (np.abs(got - ref) <= bound + 2 ** -16).all()
    assert np.sqrt(np.mean((got - ref) ** 2)) < 0.05 * np.sqrt(np.mean(ref ** 2)) + 0.01
    # M sums the unrounded p: base-2 logsumexp to fp32 accuracy
    qk_scale = float(np.float32(0.3) * np.float32(1.44269504))
    t = np.einsum("zhmd,zhnd->zhmn", qf, kf) * qk_scale
    if causal:
        t = np.where(np.tril(np.ones((N, N))) > 0, t, -np.inf)
    mx = t.max(-1, keepdims=True)
    rM = (mx[..., 0] + np.log2(np.exp2(t - mx).sum(-1))).reshape(-1, N)
    assert np.abs(M - rM).max() < 1e-5 * np.abs(rM).max() + 1e-6


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("Z,H,N,block", [(1, 2, 256, (64, 32)), (2, 1, 384, (128, 64))])
def test_attn_oracle_vs_float64(causal, Z, H, N, block):
    q, k, v = rand_qkv(Z, H, N, 64, seed=N + causal)
    o, M = oracle.attn_fwd(q, k, v, sm_scale=0.5, causal=causal, block=block)
    ro, rM = exact_attention(q, k, v, 0.5, causal)
    # p rounded to fp16 (2^-11 relative) and o to fp16: |d| <= 2^-9 for |v| <~ 2
    assert np.abs(o.view(np.float16).astype(np.float64) - ro).max() < 2 ** -9
    assert np.abs(M - rM).max() < 1e-5 * np.abs(rM).max() + 1e-6


@pytest.mark.parametrize("D,bf16", [(128, False), (64, True), (128, True)])
def test_attn_oracle_dims_and_bf16(D, bf16):
    """Head dim 128 and bf16 (p and o rounded to nearest even) against exact
    float64 attention of the same decoded inputs."""
    import torch
    rng = np.random.default_rng(D + bf16)
    x = [torch.from_numpy((rng.standard_normal((1, 2, 256, D)) * 0.5).astype(np.float32))
         for _ in range(3)]
    tdt = torch.bfloat16 if bf16 else torch.float16
    bits = [t.to(tdt).view(torch.int16).numpy().view(np.uint16) for t in x]
    qf, kf, vf = (torch.from_numpy(b.view(np.int16)).view(tdt).double().numpy() for b in bits)
    o, M = oracle.attn_fwd(*bits, sm_scale=0.5, causal=True, block=(128, 64),
                           dtype=oracle.BF16 if bf16 else oracle.F16)
    got = torch.from_numpy(o.view(np.int16)).view(tdt).double().numpy()
    N = 256
    s = np.einsum("zhmd,zhnd->zhmn", qf, kf) * 0.5
    s = np.where(np.tril(np.ones((N, N))) > 0, s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    ref = (p / p.sum(-1, keepdims=True)) @ vf
    tol = 2 ** -6 if bf16 else 2 ** -9  # p and o rounded to bf16 (8 bits) or fp16 (11)
    assert np.abs(got - ref).max() < tol, np.abs(got - ref).max()


def test_attn_loop_split_is_exact_fp8():
    import torch
    q, k, v = (torch.from_numpy(x.view(np.float16)).to(torch.float8_e5m2).view(torch.uint8)
               .numpy() for x in rand_qkv(1, 2, 512, 64, seed=4, std=1.0))
    kw = dict(sm_scale=1.3, causal=True, block=(128, 64), dtype=oracle.F8E5M2)
    o0, M0 = oracle.attn_fwd(q, k, v, mode=0, **kw)
    for mode in (1, 2):
        o1, M1 = oracle.attn_fwd(q, k, v, mode=mode, **kw)
        assert np.array_equal(o0, o1) and np.array_equal(M0.view(np.uint32), M1.view(np.uint32))


def test_attn_loop_split_is_exact():
    q, k, v = rand_qkv(1, 2, 512, 64, seed=3, std=1.0)
    for block in ((64, 32), (128, 64)):
        o0, M0 = oracle.attn_fwd(q, k, v, sm_scale=1.3, causal=True, block=block, mode=0)
        o1, M1 = oracle.attn_fwd(q, k, v, sm_scale=1.3, causal=True, block=block, mode=1)
        o2, M2 = oracle.attn_fwd(q, k, v, sm_scale=1.3, causal=True, block=block, mode=2)
        assert np.array_equal(o0, o1) and np.array_equal(M0.view(np.uint32), M1.view(np.uint32))
        assert np.array_equal(o0, o2) and np.array_equal(M0.view(np.uint32), M2.view(np.uint32))
    # and the split form is causal attention (the diagonal key included)
    ro, _ = exact_attention(q, k, v, 1.3, True)
    assert np.abs(o0.view(np.float16).astype(np.float64) - ro).max() < 2 ** -9


def test_kernel_split_is_the_loop_split_plan():
    """The kernel runs keys [0, start_m*128) unmasked and [start_m*128, +128)
    masked: the split LoopSplit computes for `start_n >= causal_start` over
    range(0, N_CTX, 64) (predicate sge, IV on the LHS)."""
    N = 2048
    for start_m in range(N // 128):
        s = tx.loop_split_plan(0, N, 64, tx.CMP_SGE, start_m * 128)
        assert s.midp == start_m * 128
        assert s.first_trips == start_m * 2 and s.second_trips == (N - start_m * 128) // 64


def test_attn_plan():
    p = tx.attn_plan(4, 32, 4096, 64, True, 1.3)
    assert (p.desc.block_m, p.desc.block_n) == (128, 64)
    assert p.grid_x == 4 * 32 * 32 and p.block_threads == 256 and p.m_blocks == 32
    assert p.flops == 0.5 * 4 * 4 * 32 * 4096 ** 2 * 64
    assert p.bytes == 4 * 4 * 32 * 4096 * 64 * 2 + 4 * 32 * 4096 * 4
    assert p.qk_scale == np.float32(np.float32(1.3) * np.float32(1.44269504))
    assert (p.desc.q_sm, p.desc.q_sh, p.desc.q_sz) == (64, 4096 * 64, 32 * 4096 * 64)
    # strided layout: [Z, N, H, D] storage viewed as [Z, H, N, D]
    p = tx.attn_plan(2, 8, 256, 64, False, 0.5,
                     strides={t: (256 * 8 * 64, 64, 8 * 64) for t in "qkvo"})
    assert p.desc.k_sm == 512 and not p.desc.causal

    def err(**kw):
        a = dict(Z=1, H=1, N_CTX=256, head_dim=64, causal=False, sm_scale=0.5)
        a.update(kw)
        with pytest.raises(tx.TxError) as e:
            tx.attn_plan(**a)
        return e.value.code
    assert err(head_dim=96) == tx.ERR_UNSUPPORTED
    # head dims: the tutorial's {16, 32, 64, 128, 256} for fp16, bf16 and fp8, at every
    # block (head dims 16 and 32 at 128 x 32: a 2 KiB K block that two of the four waves load)
    for hd in (16, 32, 64, 128, 256):
        for blk in ((128, 64), (64, 64), (64, 32), (128, 32)):
            assert tx.attn_plan(1, 1, 256, hd, True, 0.5, dtype=tx.BF16, block=blk).desc.head_dim == hd
    assert tx.attn_plan(1, 1, 256, 16, False, 0.5).flops == 4 * 256 ** 2 * 16
    assert err(head_dim=8) == tx.ERR_UNSUPPORTED
    for hd in (16, 32, 64, 128, 256):  # fp8 stages head dims 16 and 32 as 64
        for blk in ((128, 64), (64, 64)):
            p8 = tx.attn_plan(1, 2, 128, hd, False, 0.5, dtype=tx.F8E5M2, block=blk)
            assert p8.desc.q_sm == hd and p8.desc.v_sm == 128 and p8.desc.v_sh == hd * 128
            assert p8.flops == 4 * 2 * 128 ** 2 * hd
    assert err(head_dim=8, dtype=tx.F8E5M2) == tx.ERR_UNSUPPORTED
    assert err(head_dim=48, dtype=tx.F8E5M2) == tx.ERR_UNSUPPORTED
    assert err(head_dim=16, dtype=tx.F8E5M2, strides={"q": (0, 0, 8)}) == tx.ERR_INVALID
    assert err(N_CTX=200) == tx.ERR_UNSUPPORTED
    assert err(dtype=tx.F32) == tx.ERR_UNSUPPORTED
    assert tx.attn_plan(1, 1, 256, 128, True, 0.5, dtype=tx.BF16).desc.head_dim == 128
    # the tutorial's autotuned blocks: BLOCK_M 64 / 128 by BLOCK_N 32 / 64, a
    # wave per 32 query rows; N_CTX in whole BLOCK_M blocks
    for bm, bn in ((128, 64), (128, 32), (64, 64), (64, 32)):
        p = tx.attn_plan(1, 2, 192 if bm == 64 else 256, 64, True, 0.5, block=(bm, bn))
        assert (p.desc.block_m, p.desc.block_n) == (bm, bn)
        assert p.block_threads == bm // 32 * 64 and p.m_blocks == p.desc.N_CTX // bm
        assert p.grid_x == 2 * p.m_blocks
    assert err(N_CTX=192) == tx.ERR_UNSUPPORTED              # 128 rows per block by default
    assert err(N_CTX=192, block=(128, 32)) == tx.ERR_UNSUPPORTED
    for blk in ((256, 64), (64, 16), (32, 32), (128, 128)):
        assert err(block=blk) == tx.ERR_UNSUPPORTED
    # fp8 stages head dims below 64 as 64 (one byte per element); at 128 x 32
    # their 2 KiB K block is loaded by two of the four waves
    for hd, blk in ((64, (64, 32)), (16, (64, 32)), (128, (128, 32)), (256, (128, 32)),
                    (16, (128, 32)), (32, (128, 32)), (64, (128, 32))):
        p8 = tx.attn_plan(1, 2, 256, hd, True, 0.5, dtype=tx.F8E5M2, block=blk)
        assert (p8.desc.block_m, p8.desc.block_n) == blk and p8.block_threads == blk[0] // 32 * 64
    assert tx.attn_plan(1, 1, 64, 64, False, 0.5, dtype=tx.F8E5M2, block=(64, 64)).grid_x == 1
    assert err(Z=-1) == tx.ERR_INVALID
    # e5m2: one byte per element, v key-contiguous ([HEAD_DIM][N_CTX] per head)
    p8 = tx.attn_plan(4, 32, 4096, 64, False, 1.3, dtype=tx.F8E5M2)
    assert p8.bytes == 4 * 4 * 32 * 4096 * 64 + 4 * 32 * 4096 * 4
    assert (p8.desc.v_sm, p8.desc.v_sh) == (4096, 64 * 4096) and p8.desc.q_sm == 64
    assert err(dtype=tx.F8E5M2, strides={"v": (0, 0, 64)}) == tx.ERR_INVALID  # dim rows < N_CTX
    assert err(dtype=tx.F8E5M2, strides={"q": (0, 0, 72)}) == tx.ERR_INVALID  # not 16 bytes
    assert err(dtype=tx.F8E4M3) == tx.ERR_UNSUPPORTED
    assert err(sm_scale=float("nan")) == tx.ERR_INVALID
    assert err(strides={"q": (0, 0, 60)}) == tx.ERR_INVALID


def test_attention_argument_checks():
    import torch
    q = torch.zeros(1, 2, 128, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="HEAD_DIM"):
        tx.attention(q[..., :48], q[..., :48], q[..., :48], True, 0.5)
    with pytest.raises(NotImplementedError):
        tx.attention(q.float(), q.float(), q.float(), True, 0.5)
    q8 = q.to(torch.float8_e5m2)
    with pytest.raises(ValueError, match="key-contiguous"):
        tx.attention(q8, q8, q8, True, 0.5)
    with pytest.raises(ValueError, match="share one"):
        tx.attention(q, q[:, :1], q, True, 0.5)


def test_attention_signature_is_the_tutorials():
    """attention(q, k, v, causal, sm_scale, USE_TMA=True) as the tutorial's
    _attention.forward (R:pass/LoopSplit/06-fused-attention.py:583): a sixth
    positional argument is USE_TMA, and this build's extras are keyword-only."""
    import inspect
    ps = list(inspect.signature(tx.attention).parameters.values())
    assert [p.name for p in ps[:6]] == ["q", "k", "v", "causal", "sm_scale", "USE_TMA"]
    assert ps[5].default is True
    assert all(p.kind == p.KEYWORD_ONLY for p in ps[6:])
    assert {p.name for p in ps[6:]} == {"return_lse", "plan", "stream", "block"}
