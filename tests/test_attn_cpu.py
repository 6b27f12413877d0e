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


ATTN_FIXTURES = sorted(glob.glob(os.path.join(GOLDEN, "attn_*.npz")))


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
    assert err(N_CTX=200) == tx.ERR_UNSUPPORTED
    assert err(dtype=tx.F32) == tx.ERR_UNSUPPORTED
    assert tx.attn_plan(1, 1, 256, 128, True, 0.5, dtype=tx.BF16).desc.head_dim == 128
    assert err(block=(64, 32)) == tx.ERR_UNSUPPORTED
    assert err(Z=-1) == tx.ERR_INVALID
    assert err(sm_scale=float("nan")) == tx.ERR_INVALID
    assert err(strides={"q": (0, 0, 60)}) == tx.ERR_INVALID


def test_attention_argument_checks():
    import torch
    q = torch.zeros(1, 2, 128, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="HEAD_DIM"):
        tx.attention(q[..., :48], q[..., :48], q[..., :48], True, 0.5)
    with pytest.raises(NotImplementedError):
        tx.attention(q.float(), q.float(), q.float(), True, 0.5)
    with pytest.raises(ValueError, match="share one"):
        tx.attention(q, q[:, :1], q, True, 0.5)
