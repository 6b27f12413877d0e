"""Shared input generation and comparison for the parity tests.

Inputs are drawn with numpy's PCG64 from fixed seeds, so the oracle and the
GPU see identical bytes.  Seeds: A = 1, B = 2, scales = 3 (per case offset).
"""
import math
import sys

import numpy as np

import oracle


def say(*args):
    """Name the case before any GPU step, flushed (a fault loses buffered text)."""
    print("[case]", *args, flush=True)
    sys.stdout.flush()


def normal_bf16(shape, scale, seed, round_mode=oracle.ROUND_RNE):
    x = np.random.default_rng(seed).standard_normal(shape, dtype=np.float32) * np.float32(scale)
    return oracle.f32_to_bf16(x, round_mode)


def normal_f16(shape, scale, seed):
    x = np.random.default_rng(seed).standard_normal(shape, dtype=np.float32) * np.float32(scale)
    return oracle.f32_to_f16(x)


def uniform_i8(shape, seed):
    return np.random.default_rng(seed).integers(-127, 128, size=shape, dtype=np.int8)


def uniform_scales(n, seed, lo=0.001, hi=0.02):
    return np.random.default_rng(seed).uniform(lo, hi, size=n).astype(np.float32)


def fp8_block_inputs(M, N, K, seed):
    """C5 inputs: N(0,1) values, A scaled per 1x128 group, B per 128x128 block."""
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((M, K), dtype=np.float32)
    b = rng.standard_normal((K, N), dtype=np.float32)
    qa, sa = oracle.quantize_e4m3_groups(a, 1, 128)      # sa [M, K/128]
    qb, sb = oracle.quantize_e4m3_groups(b, 128, 128)    # sb [K/128, N/128]
    return qa, qb, sa, sb


def to_device(x, device):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x))
    return t.to(device)


def bits_to_f32(bits, kind):
    if kind == "bf16":
        return oracle.bf16_to_f32(bits)
    if kind == "f16":
        return oracle.f16_to_f32(bits)
    return bits.astype(np.float32)


def from_device(t):
    import torch
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def check_close(got, ref, *, atol, rtol, scale=1.0, what=""):
    """|got - ref| <= atol * scale + rtol * |ref| elementwise (fp32 arrays).

    `scale` is sqrt(K) for unnormalised inputs (outputs grow like sqrt(K)),
    1 for inputs already drawn as N(0,1)/sqrt(K).  Returns the max error.
    """
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    err = np.abs(got - ref)
    bound = atol * scale + rtol * np.abs(ref)
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(f"{what}: {bad.sum()} of {bad.size} outside tolerance; worst at {i}: "
                             f"got {got[i]!r} ref {ref[i]!r} (|d|={err[i]:.3g}, bound {bound[i]:.3g})")
    return float(err.max()) if err.size else 0.0


def k_norm(K):
    return 1.0 / math.sqrt(K)
