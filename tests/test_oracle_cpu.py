"""Pins the CPU oracle (oracle/tiled_dot.c) before anything is compared with it.

Three independent kinds of check, each able to catch a plausible mistake in
the oracle (a dropped K block, a transposed operand, a wrong mask, a wrong
rounding mode, a swapped scale index):
  1. golden fixtures written by the Triton 3.6.0 interpreter
     (tests/golden/make_golden.py), bit-exact where the inputs make every fp32
     partial sum exact, within a rigorous fp32 error bound otherwise;
  2. mathematics: int64 matmul for int8 (exact), float64 matmul with the fp32
     rounding bound for floating point, closed-form epilogues;
  3. element codecs against library conversions (numpy float16, torch bf16 and
     float8_e4m3fn) over every bit pattern or dense samples.
"""
import glob
import hashlib
import os

import numpy as np
import pytest

import oracle

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
U32 = 2.0 ** -24  # unit roundoff of fp32

OR_TYPE = {"f16": oracle.F16, "bf16": oracle.BF16, "i8": oracle.I8, "f8e4m3": oracle.F8E4M3,
           "f8e5m2": oracle.F8E5M2, "f32": oracle.F32, "i32": oracle.I32}
DECODE = {"f16": oracle.f16_to_f32, "bf16": oracle.bf16_to_f32, "f8e4m3": oracle.e4m3_to_f32,
          # e5m2 is the top byte of an fp16 (the interpreter widens it to fp16)
          "f8e5m2": lambda x: oracle.f16_to_f32(x.astype(np.uint16) << 8),
          "i8": lambda x: x.astype(np.float32)}


def load_fixture(path):
    z = np.load(path, allow_pickle=False)
    f = {k: z[k] for k in z.files}
    if "a" not in f:  # inputs regenerated from seeds (C1 recipe)
        s1, s2 = (int(s) for s in f["seeds"])
        M, N, K = int(f["M"]), int(f["N"]), int(f["K"])
        f["a"] = (np.random.default_rng(s1).standard_normal((M, K), dtype=np.float32)
                  * np.float32(K ** -0.5)).astype(np.float16).view(np.uint16)
        f["b"] = (np.random.default_rng(s2).standard_normal((K, N), dtype=np.float32)
                  * np.float32(K ** -0.5)).astype(np.float16).view(np.uint16)
    assert hashlib.sha256(f["a"].tobytes()).hexdigest() == str(f["a_sha256"])
    assert hashlib.sha256(f["b"].tobytes()).hexdigest() == str(f["b_sha256"])
    return f


# tiled-dot fixtures (the tl.dot_scaled ones, mx_*, are pinned in test_mx_oracle_cpu.py,
# attention and the e5m2 cast in test_attn_cpu.py)
FIXTURES = sorted(p for p in glob.glob(os.path.join(GOLDEN, "*.npz"))
                  if not os.path.basename(p).startswith(("mx_", "attn_", "e5m2_cast")))


def run_oracle(f, round_mode=oracle.ROUND_RTZ):
    at, ct = str(f["a_type"]), str(f["c_type"])
    sm = {0: oracle.SCALE_NONE, 1: oracle.SCALE_ROWCOL, 2: oracle.SCALE_BLOCK128}[int(f["epi"])]
    return oracle.tiled_dot(f["a"], f["b"], a_type=OR_TYPE[at], c_type=OR_TYPE[ct],
                            block=tuple(int(x) for x in f["block"]), scale_mode=sm,
                            sa=f.get("sa"), sb=f.get("sb"), round_mode=round_mode,
                            b_type=OR_TYPE[str(f.get("b_type", at))])


def fixture_output(f, c):
    """The oracle's output restricted to what the fixture stored."""
    if "c" in f:
        return c, f["c"]
    BM, BN = int(f["block"][0]), int(f["block"][1])
    got = np.stack([c[i * BM:(i + 1) * BM, j * BN:(j + 1) * BN] for i, j in f["tiles"]])
    return got, f["c_tiles"]


def as_f64(bits, kind):
    if kind in ("bf16", "f16"):
        return DECODE[kind](bits).astype(np.float64)
    return bits.astype(np.float64)


def abs_product_sum(f):
    """sum_k |a[m,k]| |b[k,n]| (with block scales applied) in float64."""
    at = str(f["a_type"])
    a = np.abs(DECODE[at](f["a"]).astype(np.float64))
    b = np.abs(DECODE[str(f.get("b_type", at))](f["b"]).astype(np.float64))
    if int(f["epi"]) == 2:
        K = a.shape[1]
        sa, sb = f["sa"].astype(np.float64), f["sb"].astype(np.float64)
        a = a * np.repeat(sa, 128, axis=1)[:, :K]
        b = b * np.repeat(np.repeat(sb, 128, axis=0), 128, axis=1)[:K, :b.shape[1]]
    return a @ b


@pytest.mark.parametrize("path", FIXTURES, ids=[os.path.basename(p)[:-4] for p in FIXTURES])
def test_golden_fixture(path):
    f = load_fixture(path)
    ct = str(f["c_type"])
    got, want = fixture_output(f, run_oracle(f))
    if bool(f["exact"]):
        assert np.array_equal(got, want), f"{np.count_nonzero(got != want)} elements differ"
        return
    g, w = as_f64(got, ct), as_f64(want, ct)
    K = int(f["K"])
    BK = int(f["block"][2])
    # fp32 accumulation in any order: |err| <= (terms per block + blocks) u sum|a||b|,
    # for each of the two implementations; plus one output rounding each.
    bound_acc = abs_product_sum(f)
    if "c_tiles" in f:
        BM, BN = int(f["block"][0]), int(f["block"][1])
        bound_acc = np.stack([bound_acc[i * BM:(i + 1) * BM, j * BN:(j + 1) * BN]
                              for i, j in f["tiles"]])
    out_u = {"f32": U32, "bf16": 2.0 ** -7, "f16": 2.0 ** -10}[ct]  # truncation: 1 ulp
    bound = 2 * (BK + K // BK + 2) * U32 * bound_acc * 1.01 + 2 * out_u * np.abs(w) + 1e-30
    assert (np.abs(g - w) <= bound).all(), float(np.max(np.abs(g - w) - bound))


def test_fixtures_present():
    names = {os.path.basename(p)[:-4] for p in FIXTURES}
    assert {"c1_fp16_512", "fp16_f32_edges_exact", "bf16_bf16_rtz_exact", "int8_i32",
            "w8a8_rowcol_rtz", "fp8_block128_f32_exact", "fp8_block128_bf16_normal",
            "fp8e5_f32_exact", "fp8e4e5_f32_exact", "fp8e5_f32_normal"} <= names


def test_e5m2_widening_matches_torch():
    """The interpreter widens fp8 to fp16; for e5m2 that is exact, so the
    oracle's decode must equal torch's float8_e5m2 -> float for every code."""
    import torch
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e5m2).float().numpy()
    got = DECODE["f8e5m2"](codes)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(got[~np.isnan(got)], ref[~np.isnan(ref)])


def test_bf16_fixture_pins_truncation():
    """The interpreter truncates fp32 -> bf16; the fixture tells RNE apart."""
    f = load_fixture(os.path.join(GOLDEN, "bf16_bf16_rtz_exact.npz"))
    rne = run_oracle(f, oracle.ROUND_RNE)
    assert not np.array_equal(rne, f["c"])
    assert np.array_equal(run_oracle(f, oracle.ROUND_RTZ), f["c"])


def test_w8a8_fixture_pins_scale_order_and_truncation():
    f = load_fixture(os.path.join(GOLDEN, "w8a8_rowcol_rtz.npz"))
    acc = (f["a"].astype(np.int64) @ f["b"].astype(np.int64)).astype(np.float32)
    v = (acc * f["sa"][:, None]) * f["sb"][None, :]          # float32 arithmetic
    assert np.array_equal(v.view(np.uint32) >> 16, f["c"].astype(np.uint32))


def test_fixture_masks_matter():
    """Edge-tile fixture: an oracle that ignored the K mask would read past K."""
    f = load_fixture(os.path.join(GOLDEN, "fp16_f32_edges_exact.npz"))
    a, b = oracle.f16_to_f32(f["a"]).astype(np.float64), oracle.f16_to_f32(f["b"]).astype(np.float64)
    assert np.array_equal((a @ b).astype(np.float32), f["c"])  # exact by construction
    assert int(f["K"]) % int(f["block"][2]) != 0 and int(f["M"]) % int(f["block"][0]) != 0


# --------------------------------------------------------------------- mathematics


@pytest.mark.parametrize("M,N,K,block", [(37, 50, 300, (16, 32, 64)), (64, 64, 128, (64, 64, 64)),
                                         (1, 300, 1000, (64, 256, 128)), (5, 7, 1, (16, 16, 16))])
def test_int8_exact(M, N, K, block):
    rng = np.random.default_rng(M * 1000 + N)
    a = rng.integers(-127, 128, (M, K), dtype=np.int8)
    b = rng.integers(-127, 128, (K, N), dtype=np.int8)
    got = oracle.tiled_dot(a, b, a_type=oracle.I8, c_type=oracle.I32, block=block)
    assert np.array_equal(got.astype(np.int64), a.astype(np.int64) @ b.astype(np.int64))


def test_int8_extremes():
    """|sum| up to 127^2 * 8192 < 2^31: no overflow at the W8A8 config's K."""
    K = 8192
    a = np.full((2, K), 127, np.int8)
    a[1] = -127
    b = np.full((K, 16), -127, np.int8)
    got = oracle.tiled_dot(a, b, a_type=oracle.I8, c_type=oracle.I32, block=(16, 16, 128))
    assert (got[0] == -127 * 127 * K).all() and (got[1] == 127 * 127 * K).all()


@pytest.mark.parametrize("kind", ["bf16", "f16"])
@pytest.mark.parametrize("M,N,K,block", [(70, 90, 200, (64, 64, 32)), (256, 128, 512, (128, 128, 64))])
def test_fp_vs_float64(kind, M, N, K, block):
    rng = np.random.default_rng(K)
    x = rng.standard_normal((M, K), dtype=np.float32)
    y = rng.standard_normal((K, N), dtype=np.float32)
    enc = oracle.f32_to_bf16 if kind == "bf16" else oracle.f32_to_f16
    dec = oracle.bf16_to_f32 if kind == "bf16" else oracle.f16_to_f32
    a, b = enc(x), enc(y)
    got = oracle.tiled_dot(a, b, a_type=OR_TYPE[kind], c_type=oracle.F32, block=block)
    A, B = dec(a).astype(np.float64), dec(b).astype(np.float64)
    exact = A @ B
    bound = (block[2] + K // block[2] + 1) * U32 * (np.abs(A) @ np.abs(B))
    assert (np.abs(got - exact) <= bound).all()
    # a transposed operand or a dropped K block is far outside that bound
    assert np.abs(got - exact).max() < 1e-3 * np.abs(exact).max()


def test_integer_valued_fp_is_exact():
    rng = np.random.default_rng(9)
    x = rng.integers(-8, 9, (33, 96)).astype(np.float32)
    y = rng.integers(-8, 9, (96, 40)).astype(np.float32)
    got = oracle.tiled_dot(oracle.f32_to_bf16(x), oracle.f32_to_bf16(y), a_type=oracle.BF16,
                           c_type=oracle.F32, block=(32, 32, 32))
    assert np.array_equal(got, x @ y)


def test_rowcol_epilogue_closed_form():
    import torch
    rng = np.random.default_rng(4)
    a = rng.integers(-127, 128, (9, 256), dtype=np.int8)
    b = rng.integers(-127, 128, (256, 48), dtype=np.int8)
    sa = rng.uniform(0.001, 0.02, 9).astype(np.float32)
    sb = rng.uniform(0.001, 0.02, 48).astype(np.float32)
    got = oracle.tiled_dot(a, b, a_type=oracle.I8, c_type=oracle.BF16, block=(16, 16, 64),
                           scale_mode=oracle.SCALE_ROWCOL, sa=sa, sb=sb, round_mode=oracle.ROUND_RNE)
    v = ((a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32) * sa[:, None]) * sb[None, :]
    want = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)


def test_block128_scales_index():
    """Each 128-K block is scaled by its own sa[m][kb] * sb[kb][n/128]: a swapped
    or shifted index changes the result by far more than rounding."""
    rng = np.random.default_rng(6)
    M, N, K = 8, 384, 384
    qa = oracle.f32_to_e4m3(rng.standard_normal((M, K), dtype=np.float32))
    qb = oracle.f32_to_e4m3(rng.standard_normal((K, N), dtype=np.float32))
    sa = rng.uniform(0.5, 2.0, (M, K // 128)).astype(np.float32)
    sb = rng.uniform(0.5, 2.0, (K // 128, N // 128)).astype(np.float32)
    got = oracle.tiled_dot(qa, qb, a_type=oracle.F8E4M3, c_type=oracle.F32, block=(16, 128, 128),
                           scale_mode=oracle.SCALE_BLOCK128, sa=sa, sb=sb)
    A, B = oracle.e4m3_to_f32(qa).astype(np.float64), oracle.e4m3_to_f32(qb).astype(np.float64)
    want = np.zeros((M, N))
    for kb in range(K // 128):
        part = A[:, kb * 128:(kb + 1) * 128] @ B[kb * 128:(kb + 1) * 128]
        want += part * sa[:, kb:kb + 1] * np.repeat(sb[kb], 128)[None, :]
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()


def test_tile_subset_leaves_other_tiles():
    rng = np.random.default_rng(2)
    a = rng.integers(-5, 6, (100, 64), dtype=np.int8)
    b = rng.integers(-5, 6, (64, 100), dtype=np.int8)
    out = np.full((100, 100), 12345, np.int32)
    oracle.tiled_dot(a, b, a_type=oracle.I8, c_type=oracle.I32, block=(32, 32, 64), tiles=(1, 2),
                     out=out)
    full = a.astype(np.int64) @ b.astype(np.int64)
    assert np.array_equal(out[:32, 32:64], full[:32, 32:64])
    assert (out[:32, :32] == 12345).all() and (out[32:, :] == 12345).all()


def test_rejects_bad_arguments():
    a = np.zeros((4, 4), np.int8)
    with pytest.raises(ValueError):
        oracle.tiled_dot(a, a, a_type=oracle.I8, c_type=oracle.I32, block=(0, 16, 16))
    with pytest.raises(ValueError):  # block scales need 128-wide K blocks
        oracle.tiled_dot(a, a, a_type=oracle.F8E4M3, c_type=oracle.F32, block=(16, 16, 64),
                         scale_mode=oracle.SCALE_BLOCK128, sa=np.ones((4, 1), np.float32),
                         sb=np.ones((1, 1), np.float32))


# --------------------------------------------------------------------- codecs


def test_bf16_decode_all_patterns():
    import torch
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    ours = oracle.bf16_to_f32(h)
    ref = torch.from_numpy(h.view(np.int16)).view(torch.bfloat16).float().numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def _f32_samples():
    rng = np.random.default_rng(11)
    u = rng.integers(0, 1 << 32, 200000, dtype=np.uint64).astype(np.uint32)
    ties = (rng.integers(0, 1 << 16, 5000, dtype=np.uint32) << 16) | 0x8000  # bf16 ties
    specials = np.array([0, 0x80000000, 0x7f800000, 0xff800000, 0x7f7fffff, 0x00000001,
                         0x3f808000, 0x3f818000, 0x477fe000, 0x477ff000, 0x33000000], np.uint32)
    return np.concatenate([u, ties, specials]).view(np.float32)


def test_bf16_encode_rne_vs_torch():
    import torch
    x = _f32_samples()
    ours = oracle.f32_to_bf16(x, oracle.ROUND_RNE)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(ours[~nan], ref[~nan])
    assert (oracle.bf16_to_f32(ours[nan]) != oracle.bf16_to_f32(ours[nan])).all()


def test_bf16_encode_rtz_is_truncation():
    x = _f32_samples()
    ours = oracle.f32_to_bf16(x, oracle.ROUND_RTZ)
    nan = np.isnan(x)
    assert np.array_equal(ours[~nan], (x.view(np.uint32)[~nan] >> 16).astype(np.uint16))


def test_f16_codec_vs_numpy():
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    ours = oracle.f16_to_f32(h)
    nan = np.isnan(ref)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    rng = np.random.default_rng(3)
    x = np.concatenate([_f32_samples(), rng.uniform(-7e4, 7e4, 100000).astype(np.float32),
                        rng.uniform(-1e-4, 1e-4, 100000).astype(np.float32),
                        (np.arange(-2048, 2048) * 2.0 ** -25).astype(np.float32)])
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    got = oracle.f32_to_f16(x)
    ok = ~np.isnan(x)
    assert np.array_equal(got[ok], want[ok])


def test_e4m3_decode_vs_torch():
    import torch
    q = np.arange(256, dtype=np.uint8)
    ours = oracle.e4m3_to_f32(q)
    ref = torch.from_numpy(q).view(torch.float8_e4m3fn).float().numpy()
    finite = ~np.isnan(ref)
    assert finite.sum() == 254  # 0x7f and 0xff are NaN in e4m3fn
    assert np.array_equal(ours[finite], ref[finite])
    # the interpreter's generic converter reads the NaN codes as +-480
    assert ours[0x7F] == 480.0 and ours[0xFF] == -480.0
    assert ours[0x7E] == 448.0 and ours[0x01] == 2.0 ** -9


def test_e4m3_encode_vs_torch():
    import torch
    rng = np.random.default_rng(8)
    x = np.concatenate([rng.uniform(-448, 448, 200000), rng.uniform(-0.05, 0.05, 100000),
                        oracle.e4m3_to_f32(np.arange(256, dtype=np.uint8)[:0x7e]).astype(np.float64)
                        ]).astype(np.float32)
    ours = oracle.f32_to_e4m3(x)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, ref)
    sat = oracle.f32_to_e4m3(np.array([500.0, -1e6, 449.0], np.float32))
    assert list(sat) == [0x7E, 0xFE, 0x7E]  # saturates to +-448


def test_group_quantisation():
    rng = np.random.default_rng(12)
    x = rng.standard_normal((6, 300), dtype=np.float32)
    x[2, 128:256] = 0
    q, s = oracle.quantize_e4m3_groups(x, 1, 128)
    assert s.shape == (6, 3)
    for i in range(6):
        for j in range(3):
            blk = x[i, j * 128:(j + 1) * 128]
            amax = np.abs(blk).max()
            assert s[i, j] == (np.float32(amax) / np.float32(448) if amax > 0 else 1.0)
    back = oracle.e4m3_to_f32(q) * np.repeat(s, 128, axis=1)[:, :300]
    assert np.abs(back - x).max() <= np.abs(x).max() * 2.0 ** -4
