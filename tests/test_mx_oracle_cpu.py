"""Pins the CPU oracle's tl.dot_scaled (oracle_dot_scaled in oracle/tiled_dot.c).

The interpreter has no dot_scaled, so no single source gives its output; the
restatement is pinned from several independent sides, each able to catch a
plausible mistake (a wrong nibble order, a transposed rhs_scale, a scale
applied to the wrong 32-element group, a NaN rule dropped):
  1. codecs: e4m3 / e5m2 / e8m0 against torch's float8_e4m3fn, float8_e5m2
     and float8_e8m0fnu over every code; e2m1 against the OCP table and the
     e4m3 encoding of the same values;
  2. reductions to already-pinned functions: unit scales give the tiled fp8
     dot (pinned by the interpreter's tl.dot fixtures), and e2m1 operands give
     exactly what their e4m3 re-encoding gives (fp8 path: no packing);
  3. invariants: +1 on every scale of a row (column) doubles that row
     (column); +1 on one group adds exactly that group's terms; NaN scales and
     NaN codes poison exactly their rows / columns;
  4. brute force in numpy float64 on tiny shapes;
  5. golden fixtures from the Triton interpreter running dot_scaled's upcast
     form (tests/golden/make_golden.py: decode, times exp2(s - 127), tl.dot).
"""
import glob
import os

import numpy as np
import pytest
import torch

import oracle

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FMT = {"e4m3": oracle.F8E4M3, "e5m2": oracle.F8E5M2, "e2m1": oracle.F4E2M1}
U32 = 2.0 ** -24
CODES = np.arange(256, dtype=np.uint8)


def same(x, y):
    """Equal as float64, NaN where the other is NaN."""
    x, y = np.asarray(x, np.float64), np.asarray(y, np.float64)
    return np.array_equal(np.isnan(x), np.isnan(y)) and np.array_equal(x[~np.isnan(x)],
                                                                        y[~np.isnan(y)])


def test_e8m0_decode_matches_torch():
    ref = torch.from_numpy(CODES).view(torch.float8_e8m0fnu).to(torch.float64).numpy()
    assert same(oracle.mx_decode(CODES, oracle.E8M0), ref)
    assert oracle.mx_decode(np.array([0, 127, 254], np.uint8), oracle.E8M0).tolist() == \
        [2.0 ** -127, 1.0, 2.0 ** 127]


@pytest.mark.parametrize("fmt,tdt", [(oracle.F8E4M3, torch.float8_e4m3fn),
                                     (oracle.F8E5M2, torch.float8_e5m2)])
def test_fp8_decode_matches_torch(fmt, tdt):
    ref = torch.from_numpy(CODES).view(tdt).to(torch.float64).numpy()
    assert same(oracle.mx_decode(CODES, fmt), ref)


def test_e2m1_decode():
    # OCP MX v1.0 FP4 E2M1 table: 0, 0.5, 1, 1.5, 2, 3, 4, 6 and negatives
    table = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    v = oracle.mx_decode(np.arange(16, dtype=np.uint8), oracle.F4E2M1)
    assert v[:8].tolist() == table
    assert v[8:].tolist() == [-x for x in table]
    # every e2m1 value is an e4m3 value: the fp8 encoding decodes back exactly
    q = torch.from_numpy(v.astype(np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(oracle.mx_decode(q, oracle.F8E4M3), v)


def pack_e2m1(codes, axis):
    lo = np.take(codes, np.arange(0, codes.shape[axis], 2), axis=axis)
    hi = np.take(codes, np.arange(1, codes.shape[axis], 2), axis=axis)
    return (lo | (hi << 4)).astype(np.uint8)


def exact_codes(rng, shape, fmt):
    """Codes whose scaled products and sums stay exact in fp32."""
    if fmt == oracle.F4E2M1:
        return rng.integers(0, 16, size=shape, dtype=np.uint8)
    if fmt == oracle.F8E4M3:
        return (rng.integers(0, 2, size=shape) << 7 | rng.integers(5, 9, size=shape) << 3
                | rng.integers(0, 8, size=shape)).astype(np.uint8)
    return (rng.integers(0, 2, size=shape) << 7 | rng.integers(13, 17, size=shape) << 2
            | rng.integers(0, 4, size=shape)).astype(np.uint8)


def brute(ac, sa, fa, bc, sb, fb):
    """numpy float64: decode unpacked codes, scale per 32 along K, matmul."""
    K = ac.shape[1]
    g = np.arange(K) // 32
    a = oracle.mx_decode(ac, fa) * np.exp2(sa[:, g].astype(np.float64) - 127)
    b = oracle.mx_decode(bc, fb) * np.exp2(sb[:, g].T.astype(np.float64) - 127)
    return (a @ b).astype(np.float32)


def run(ac, sa, fa, bc, sb, fb, **kw):
    a = pack_e2m1(ac, 1) if fa == oracle.F4E2M1 else ac
    b = pack_e2m1(bc, 0) if fb == oracle.F4E2M1 else bc
    return oracle.dot_scaled(a, sa, fa, b, sb, fb, K=ac.shape[1], **kw)


@pytest.mark.parametrize("fa,fb", [(oracle.F8E4M3, oracle.F8E4M3), (oracle.F8E5M2, oracle.F8E4M3),
                                   (oracle.F4E2M1, oracle.F4E2M1)])
def test_brute_force_tiny(fa, fb):
    rng = np.random.default_rng(7)
    M, N, K = 5, 7, 96  # N != K/32: a transposed rhs_scale cannot pass
    ac, bc = exact_codes(rng, (M, K), fa), exact_codes(rng, (K, N), fb)
    sa = rng.integers(120, 135, size=(M, K // 32)).astype(np.uint8)
    sb = rng.integers(120, 135, size=(N, K // 32)).astype(np.uint8)
    assert np.array_equal(run(ac, sa, fa, bc, sb, fb), brute(ac, sa, fa, bc, sb, fb))


def test_unit_scales_reduce_to_tiled_fp8_dot():
    rng = np.random.default_rng(8)
    M, N, K = 33, 40, 256
    ac, bc = exact_codes(rng, (M, K), oracle.F8E4M3), exact_codes(rng, (K, N), oracle.F8E4M3)
    ones_a = np.full((M, K // 32), 127, np.uint8)
    ones_b = np.full((N, K // 32), 127, np.uint8)
    got = run(ac, ones_a, oracle.F8E4M3, bc, ones_b, oracle.F8E4M3)
    ref = oracle.tiled_dot(ac, bc, a_type=oracle.F8E4M3, c_type=oracle.F32, block=(32, 32, 64))
    assert np.array_equal(got, ref)


def test_e2m1_equals_its_e4m3_reencoding():
    rng = np.random.default_rng(9)
    M, N, K = 24, 20, 192
    ac = rng.integers(0, 16, size=(M, K), dtype=np.uint8)
    bc = rng.integers(0, 16, size=(K, N), dtype=np.uint8)
    sa = rng.integers(110, 140, size=(M, K // 32)).astype(np.uint8)
    sb = rng.integers(110, 140, size=(N, K // 32)).astype(np.uint8)

    def to_e4m3(c):
        v = oracle.mx_decode(c, oracle.F4E2M1).astype(np.float32)
        return torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()

    fp4 = run(ac, sa, oracle.F4E2M1, bc, sb, oracle.F4E2M1)
    fp8 = run(to_e4m3(ac), sa, oracle.F8E4M3, to_e4m3(bc), sb, oracle.F8E4M3)
    assert np.array_equal(fp4, fp8)
    # a swapped nibble order would not pass
    swapped = run(ac.reshape(M, K // 2, 2)[:, :, ::-1].reshape(M, K), sa, oracle.F4E2M1,
                  bc, sb, oracle.F4E2M1)
    assert not np.array_equal(swapped, fp8)


def test_scale_steps():
    rng = np.random.default_rng(10)
    M, N, K = 6, 9, 128
    f = oracle.F8E4M3

    def narrow(shape):  # e4m3 values +-[1, 2): with scales 2^-1..2^1 every sum is exact
        return (rng.integers(0, 2, size=shape) << 7 | 7 << 3
                | rng.integers(0, 8, size=shape)).astype(np.uint8)

    ac, bc = narrow((M, K)), narrow((K, N))
    sa = rng.integers(126, 129, size=(M, K // 32)).astype(np.uint8)
    sb = rng.integers(126, 129, size=(N, K // 32)).astype(np.uint8)
    base = run(ac, sa, f, bc, sb, f)
    sa2 = sa.copy()
    sa2[2] += 1
    c = run(ac, sa2, f, bc, sb, f)
    assert np.array_equal(c[2], 2 * base[2]) and np.array_equal(np.delete(c, 2, 0),
                                                                 np.delete(base, 2, 0))
    sb2 = sb.copy()
    sb2[4] += 1
    c = run(ac, sa, f, bc, sb2, f)
    assert np.array_equal(c[:, 4], 2 * base[:, 4]) and np.array_equal(np.delete(c, 4, 1),
                                                                       np.delete(base, 4, 1))
    # +1 on group 1 of row 3 adds exactly that group's terms
    sa3 = sa.copy()
    sa3[3, 1] += 1
    only = ac.copy()
    only[:, :32] = 0
    only[:, 64:] = 0
    c = run(ac, sa3, f, bc, sb, f)
    assert np.array_equal(c[3], base[3] + run(only, sa, f, bc, sb, f)[3])


def test_nan_rules():
    rng = np.random.default_rng(11)
    M, N, K = 4, 5, 64
    f = oracle.F8E4M3
    ac, bc = exact_codes(rng, (M, K), f), exact_codes(rng, (K, N), f)
    sa = np.full((M, K // 32), 127, np.uint8)
    sb = np.full((N, K // 32), 127, np.uint8)
    sa[1, 1] = 255
    sb[3, 0] = 255
    c = run(ac, sa, f, bc, sb, f)
    nan = np.zeros((M, N), bool)
    nan[1, :] = True
    nan[:, 3] = True
    assert np.array_equal(np.isnan(c), nan)
    ac2 = ac.copy()
    ac2[2, 40] = 0x7F  # e4m3fn NaN code
    c = run(ac2, np.full_like(sa, 127), f, bc, np.full_like(sb, 127), f)
    assert np.isnan(c[2]).all() and not np.isnan(np.delete(c, 2, 0)).any()


MX_FIXTURES = sorted(glob.glob(os.path.join(GOLDEN, "mx_*.npz")))


@pytest.mark.parametrize("path", MX_FIXTURES, ids=[os.path.basename(p)[:-4] for p in MX_FIXTURES])
def test_golden_fixture_mx(path):
    z = np.load(path, allow_pickle=False)
    fa, fb, K = FMT[str(z["a_fmt"])], FMT[str(z["b_fmt"])], int(z["K"])
    got = oracle.dot_scaled(z["a"], z["sa"], fa, z["b"], z["sb"], fb, K=K)
    want = z["c"]
    if bool(z["exact"]):
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        return
    # the interpreter sums in fp32 (np.matmul): |err| <= K u sum|a||b|, the
    # oracle rounds the exact sum once (u |c|)
    def deq(codes, s, f, axis):
        if f == oracle.F4E2M1:
            lo, hi = codes & 15, codes >> 4
            codes = np.stack([lo, hi], axis=axis + 1).reshape(
                (codes.shape[0] * 2, -1) if axis == 0 else (codes.shape[0], -1))
        return codes
    ac = deq(z["a"], z["sa"], fa, 1)
    bc = deq(z["b"], z["sb"], fb, 0)
    g = np.arange(K) // 32
    a = np.abs(oracle.mx_decode(ac, fa) * np.exp2(z["sa"][:, g].astype(np.float64) - 127))
    b = np.abs(oracle.mx_decode(bc, fb) * np.exp2(z["sb"][:, g].T.astype(np.float64) - 127))
    bound = (K + 1) * U32 * (a @ b) + 1e-30
    assert (np.abs(got.astype(np.float64) - want) <= bound).all()


def _e4m3_codes(rng, shape):
    c = rng.integers(0, 256, size=shape).astype(np.uint8)
    return np.where((c & 0x7F) == 0x7F, c & 0xF0, c).astype(np.uint8)


@pytest.mark.parametrize("side", ["a", "b"])
@pytest.mark.parametrize("fmt", [oracle.F4E2M1, oracle.F8E5M2])
def test_bf16_side_reduces_to_mx(side, fmt):
    """tl.dot_scaled with a bf16 operand (T:language/core.py:2072-2076):
    when the bf16 values are e4m3 values and the MX side's upcast is exact
    (moderate scales), the result equals the all-MX dot with e4m3 codes and
    unit scales in place of the bf16 operand, bit for bit."""
    rng = np.random.default_rng(5 + (side == "b"))
    M, N, K = 24, 40, 96
    e4 = _e4m3_codes(rng, (M, K) if side == "a" else (K, N))
    bf = torch.from_numpy(e4).view(torch.float8_e4m3fn).float().to(torch.bfloat16) \
        .view(torch.int16).numpy().view(np.uint16)
    rows = K if fmt != oracle.F4E2M1 else K // 2
    if side == "a":  # A bf16, B MX
        c = rng.integers(0, 16, size=(K, N)).astype(np.uint8) if fmt == oracle.F4E2M1 else \
            rng.integers(0, 0x7C, size=(K, N)).astype(np.uint8)
        b = (c[0::2] | (c[1::2] << 4)).astype(np.uint8) if fmt == oracle.F4E2M1 else c
        assert b.shape[0] == rows
        sb = rng.integers(117, 138, size=(N, K // 32)).astype(np.uint8)
        got = oracle.dot_scaled(bf, None, oracle.BF16, b, sb, fmt, K=K)
        want = oracle.dot_scaled(e4, np.full((M, K // 32), 127, np.uint8), oracle.F8E4M3,
                                 b, sb, fmt, K=K)
    else:  # A MX, B bf16
        c = rng.integers(0, 16, size=(M, K)).astype(np.uint8) if fmt == oracle.F4E2M1 else \
            rng.integers(0, 0x7C, size=(M, K)).astype(np.uint8)
        a = (c[:, 0::2] | (c[:, 1::2] << 4)).astype(np.uint8) if fmt == oracle.F4E2M1 else c
        sa = rng.integers(117, 138, size=(M, K // 32)).astype(np.uint8)
        got = oracle.dot_scaled(a, sa, fmt, bf, None, oracle.BF16, K=K)
        want = oracle.dot_scaled(a, sa, fmt, e4, np.full((N, K // 32), 127, np.uint8),
                                 oracle.F8E4M3, K=K)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_bf16_side_upcast_rounds_to_bf16():
    """The MX side is rounded to bf16 before the products: an e4m3 subnormal
    7 * 2^-9 scaled by 2^-127 is 7 * 2^-136, below bf16's 2^-133 quantum, so
    it becomes torch's bf16 of that value (2^-133); 448 * 2^127 overflows to
    inf; scale 0xFF is NaN."""
    K = 32
    one = torch.tensor([1.0], dtype=torch.bfloat16).view(torch.int16).numpy().view(np.uint16)[0]
    a = np.zeros((1, K), np.uint16)
    a[0, 3] = one
    b = np.zeros((K, 3), np.uint8)
    b[3] = [0x07, 0x7E, 0x38]  # e4m3: 7 * 2^-9, 448, 1.0
    sb = np.array([[0], [254], [255]], np.uint8)
    c = oracle.dot_scaled(a, None, oracle.BF16, b, sb, oracle.F8E4M3, K=K)[0]
    want0 = torch.tensor([7 * 2.0 ** -136], dtype=torch.float32).to(torch.bfloat16).float().item()
    assert want0 == 2.0 ** -133 and c[0] == np.float32(want0)
    assert np.isposinf(c[1]) and np.isnan(c[2])


def test_nv16_power_of_two_scales_equal_mx32():
    """e4m3 scales per 16 K (tl.dot_scaled's fp8e4nv scale tensors): with
    power-of-two e4m3 scales 2^k (code (k + 7) << 3), equal on both 16-halves
    of every 32-group, the result equals the MX dot with e8m0 127 + k, bit
    for bit (the e2m1 x e4m3 upcast is exact)."""
    rng = np.random.default_rng(12)
    M, N, K = 24, 40, 128
    ac = rng.integers(0, 16, size=(M, K)).astype(np.uint8)
    bc = rng.integers(0, 16, size=(K, N)).astype(np.uint8)
    a = (ac[:, 0::2] | (ac[:, 1::2] << 4)).astype(np.uint8)
    b = (bc[0::2] | (bc[1::2] << 4)).astype(np.uint8)
    ka = rng.integers(-6, 9, size=(M, K // 32))
    kb = rng.integers(-6, 9, size=(N, K // 32))
    nv_a = np.repeat(((ka + 7) << 3).astype(np.uint8), 2, axis=1)
    nv_b = np.repeat(((kb + 7) << 3).astype(np.uint8), 2, axis=1)
    got = oracle.dot_scaled(a, nv_a, oracle.F4E2M1, b, nv_b, oracle.F4E2M1, K=K, nv16=True)
    want = oracle.dot_scaled(a, (127 + ka).astype(np.uint8), oracle.F4E2M1, b,
                             (127 + kb).astype(np.uint8), oracle.F4E2M1, K=K)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # a non-power-of-two scale (1.5 = code 0x3C) scales its 16 terms exactly
    one = np.full_like(nv_a, 0x38)
    c1 = oracle.dot_scaled(a, one, oracle.F4E2M1, b, np.full_like(nv_b, 0x38), oracle.F4E2M1,
                           K=K, nv16=True)
    c15 = oracle.dot_scaled(a, np.full_like(nv_a, 0x3C), oracle.F4E2M1, b,
                            np.full_like(nv_b, 0x38), oracle.F4E2M1, K=K, nv16=True)
    assert np.array_equal(c15, (c1.astype(np.float64) * 1.5).astype(np.float32))


@pytest.mark.parametrize("K", [16, 48, 80])
def test_nv16_k_a_multiple_of_16(K):
    """e4m3 scales per 16 need K % 16 == 0 only (an odd number of 16-groups included):
    the oracle equals a float64 brute force of decode(e2m1) * decode(e4m3 scale) per 16,
    summed and rounded once to fp32, bit for bit."""
    import torch
    rng = np.random.default_rng(K)
    M, N = 5, 7
    ac = rng.integers(0, 16, size=(M, K)).astype(np.uint8)
    bc = rng.integers(0, 16, size=(K, N)).astype(np.uint8)
    a = (ac[:, 0::2] | (ac[:, 1::2] << 4)).astype(np.uint8)
    b = (bc[0::2] | (bc[1::2] << 4)).astype(np.uint8)
    sa = rng.integers(0x20, 0x50, size=(M, K // 16)).astype(np.uint8)
    sb = rng.integers(0x20, 0x50, size=(N, K // 16)).astype(np.uint8)
    got = oracle.dot_scaled(a, sa, oracle.F4E2M1, b, sb, oracle.F4E2M1, K=K, nv16=True)
    dec4 = lambda c: torch.from_numpy(c).view(torch.float8_e4m3fn).double().numpy()
    g = np.arange(K) // 16
    fa = oracle.mx_decode(ac, oracle.F4E2M1) * dec4(sa)[:, g]
    fb = oracle.mx_decode(bc, oracle.F4E2M1) * dec4(sb)[:, g].T
    want = (fa @ fb).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
