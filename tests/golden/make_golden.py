"""Write the golden fixtures in this directory with the Triton interpreter.

    TRITON_INTERPRET=1 python tests/golden/make_golden.py

Runs in the build container only (needs the third-party triton-rocm 3.6.0
package; nothing on the GPU box imports triton).  Each fixture is an .npz of
raw element bits: the inputs, the launch parameters and the interpreter's
output for one tiled-dot kernel, the kernel a Triton user writes around
`tl.dot` (the reference's call sites: R:pass/LoopSplit/06-fused-attention.py:63,85):

    acc = zeros([BM, BN], fp32 | int32)
    for k0 in range(0, K, BK):
        a = tl.load(A[m, k0 + k], mask=in-bounds, other=0)
        b = tl.load(B[k0 + k, n], mask=in-bounds, other=0)
        acc = tl.dot(a, b, acc)                 # bf16 tiles .to(fp32) first
    tl.store(C[m, n], epilogue(acc).to(OUT), mask=in-bounds)

Interpreter facts the fixtures exercise (third-party source, read as text):
  * grid order x -> y -> z, one program at a time (triton/runtime/interpreter.py:1353-1357);
  * masked loads return `other` (:449-455);
  * tl.dot = np.matmul(a, b, dtype=acc) + acc, fp8 widened to fp16 first (:630-637);
  * bf16 is stored as uint16 (:186-187), so bf16 tiles are cast to fp32 before
    tl.dot; fp32 -> bf16 casts truncate (cast_impl, :461-467, rounding None);
  * fp32 -> fp16 casts are numpy astype (round to nearest even).

tl.dot_scaled (MX) fixtures: the interpreter has no dot_scaled, so mx_dot_kernel
runs the form it reduces to, each operand upcast then tl.dot in fp32
(T:language/semantic.py:1611-1665 for the operand and scale shapes): codes are
loaded as uint8, decoded with the OCP e4m3 / e5m2 / e2m1 formulas (e2m1
unpacked low nibble first along K), multiplied by exp2(scale - 127) per 32
elements of K (rhs_scale indexed [n][k // 32]), and accumulated by tl.dot.

attn_* fixtures: attn_fwd_kernel below follows the forward of the reference's
fused-attention tutorial step for step (R:pass/LoopSplit/06-fused-attention.py
:44-93 _attn_fwd_inner, :181-239 _attn_fwd) with plain pointers in place of
block pointers: one loop over all keys with the on-band branch
`start_n >= causal_start`, exp2 softmax with qk_scale = sm_scale * 1.44269504,
p.to(fp16) @ v, M = m_i + log2(l_i), o = acc / l_i.  Inputs N(0, 0.5) fp16
as in the tutorial's test_op.

"dyadic" fixtures draw small multiples of a power of two, so every product and
partial sum is exact in fp32: the fp32 accumulator is then independent of the
summation order, and any correct implementation must match it bit for bit.
"""
import hashlib
import os
import sys

os.environ["TRITON_INTERPRET"] = "1"

import numpy as np  # noqa: E402
import torch  # noqa: E402
import triton  # noqa: E402
import triton.language as tl  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))

EPI_NONE, EPI_ROWCOL, EPI_BLOCK128 = 0, 1, 2


@triton.jit
def tiled_dot_kernel(a_ptr, b_ptr, c_ptr, sa_ptr, sb_ptr, M, N, K, sa_ld, sb_ld,
                     BM: tl.constexpr, BN: tl.constexpr, BK: tl.constexpr,
                     WIDEN: tl.constexpr, INT_ACC: tl.constexpr, EPI: tl.constexpr,
                     OUT: tl.constexpr, MASK: tl.constexpr):
    pid_m = tl.program_id(0)
    pid_n = tl.program_id(1)
    rm = pid_m * BM + tl.arange(0, BM)
    rn = pid_n * BN + tl.arange(0, BN)
    rk = tl.arange(0, BK)
    if INT_ACC:
        acc = tl.zeros((BM, BN), dtype=tl.int32)
    else:
        acc = tl.zeros((BM, BN), dtype=tl.float32)
    for k0 in range(0, K, BK):
        kk = k0 + rk
        if MASK:
            a = tl.load(a_ptr + rm[:, None] * K + kk[None, :],
                        mask=(rm[:, None] < M) & (kk[None, :] < K), other=0)
            b = tl.load(b_ptr + kk[:, None] * N + rn[None, :],
                        mask=(kk[:, None] < K) & (rn[None, :] < N), other=0)
        else:  # whole tiles only (the interpreter cannot fill fp8 `other`)
            a = tl.load(a_ptr + rm[:, None] * K + kk[None, :])
            b = tl.load(b_ptr + kk[:, None] * N + rn[None, :])
        if WIDEN:
            a = a.to(tl.float32)
            b = b.to(tl.float32)
        if EPI == 2:
            part = tl.dot(a, b, tl.zeros((BM, BN), dtype=tl.float32))
            s_a = tl.load(sa_ptr + rm * sa_ld + k0 // BK, mask=rm < M, other=0.0)
            s_b = tl.load(sb_ptr + (k0 // BK) * sb_ld + rn // 128, mask=rn < N, other=0.0)
            acc = acc + part * s_a[:, None] * s_b[None, :]
        elif INT_ACC:
            acc = tl.dot(a, b, acc, out_dtype=tl.int32)
        else:
            acc = tl.dot(a, b, acc)
    if EPI == 1:
        s_a = tl.load(sa_ptr + rm, mask=rm < M, other=0.0)
        s_b = tl.load(sb_ptr + rn, mask=rn < N, other=0.0)
        res = acc.to(tl.float32) * s_a[:, None] * s_b[None, :]
    else:
        res = acc
    tl.store(c_ptr + rm[:, None] * N + rn[None, :], res.to(OUT),
             mask=(rm[:, None] < M) & (rn[None, :] < N))


@triton.jit
def _mx_decode(c, FMT: tl.constexpr):
    """OCP element value of uint8 codes (as int32): 0 e4m3, 1 e5m2, 4 e2m1."""
    if FMT == 0:
        e = (c >> 3) & 15
        m = (c & 7).to(tl.float32)
        mag = tl.where(e == 0, m * 0.001953125,
                       (1.0 + m * 0.125) * tl.exp2((e - 7).to(tl.float32)))
        sgn = c >> 7
    elif FMT == 1:
        e = (c >> 2) & 31
        m = (c & 3).to(tl.float32)
        mag = tl.where(e == 0, m * 0.0000152587890625,
                       (1.0 + m * 0.25) * tl.exp2((e - 15).to(tl.float32)))
        sgn = c >> 7
    else:
        e = (c >> 1) & 3
        m = (c & 1).to(tl.float32)
        mag = tl.where(e == 0, m * 0.5, (1.0 + m * 0.5) * tl.exp2((e - 1).to(tl.float32)))
        sgn = (c >> 3) & 1
    return tl.where(sgn != 0, -mag, mag)


@triton.jit
def mx_dot_kernel(a_ptr, b_ptr, sa_ptr, sb_ptr, c_ptr, M, N, K,
                  BM: tl.constexpr, BN: tl.constexpr, BK: tl.constexpr,
                  FA: tl.constexpr, FB: tl.constexpr):
    pid_m = tl.program_id(0)
    pid_n = tl.program_id(1)
    rm = pid_m * BM + tl.arange(0, BM)
    rn = pid_n * BN + tl.arange(0, BN)
    rk = tl.arange(0, BK)
    G = K // 32
    acc = tl.zeros((BM, BN), dtype=tl.float32)
    for k0 in range(0, K, BK):
        kk = k0 + rk
        am = (rm[:, None] < M) & (kk[None, :] < K)
        bm = (kk[:, None] < K) & (rn[None, :] < N)
        if FA == 4:
            ab = tl.load(a_ptr + rm[:, None] * (K // 2) + kk[None, :] // 2, mask=am, other=0)
            ac = (ab.to(tl.int32) >> ((kk[None, :] % 2) * 4)) & 15
        else:
            ac = tl.load(a_ptr + rm[:, None] * K + kk[None, :], mask=am, other=0).to(tl.int32)
        if FB == 4:
            bb = tl.load(b_ptr + (kk[:, None] // 2) * N + rn[None, :], mask=bm, other=0)
            bc = (bb.to(tl.int32) >> ((kk[:, None] % 2) * 4)) & 15
        else:
            bc = tl.load(b_ptr + kk[:, None] * N + rn[None, :], mask=bm, other=0).to(tl.int32)
        sa = tl.load(sa_ptr + rm[:, None] * G + kk[None, :] // 32, mask=am, other=127)
        sb = tl.load(sb_ptr + rn[None, :] * G + kk[:, None] // 32, mask=bm, other=127)
        a = _mx_decode(ac, FA) * tl.exp2(sa.to(tl.float32) - 127.0)
        b = _mx_decode(bc, FB) * tl.exp2(sb.to(tl.float32) - 127.0)
        acc = tl.dot(a, b, acc)
    tl.store(c_ptr + rm[:, None] * N + rn[None, :], acc,
             mask=(rm[:, None] < M) & (rn[None, :] < N))


@triton.jit
def attn_fwd_kernel(Q, K, V, sm_scale, M, Out, N_CTX, H,
                    HEAD_DIM: tl.constexpr, BLOCK_M: tl.constexpr, BLOCK_N: tl.constexpr,
                    CAUSAL: tl.constexpr):
    start_m = tl.program_id(0)
    off_hz = tl.program_id(1)
    base = off_hz.to(tl.int64) * N_CTX * HEAD_DIM
    offs_m = start_m * BLOCK_M + tl.arange(0, BLOCK_M)
    offs_n = tl.arange(0, BLOCK_N)
    offs_d = tl.arange(0, HEAD_DIM)
    m_i = tl.zeros([BLOCK_M], dtype=tl.float32) - float("inf")
    l_i = tl.zeros([BLOCK_M], dtype=tl.float32) + 1.0
    acc = tl.zeros([BLOCK_M, HEAD_DIM], dtype=tl.float32)
    qk_scale = sm_scale
    qk_scale *= 1.44269504
    q = tl.load(Q + base + offs_m[:, None] * HEAD_DIM + offs_d[None, :])
    if CAUSAL:
        causal_start = start_m * BLOCK_M
    else:
        causal_start = N_CTX
    for start_n in range(0, N_CTX, BLOCK_N):
        kt = tl.load(K + base + (start_n + offs_n)[None, :] * HEAD_DIM + offs_d[:, None])
        qk = tl.dot(q, kt)
        if start_n >= causal_start:
            mask = offs_m[:, None] >= (start_n + offs_n[None, :])
            qk = qk * qk_scale + tl.where(mask, 0, -1.0e6)
            m_ij = tl.maximum(m_i, tl.max(qk, 1))
            qk -= m_ij[:, None]
        else:
            m_ij = tl.maximum(m_i, tl.max(qk, 1) * qk_scale)
            qk = qk * qk_scale - m_ij[:, None]
        p = tl.math.exp2(qk)
        l_ij = tl.sum(p, 1)
        alpha = tl.math.exp2(m_i - m_ij)
        l_i = l_i * alpha + l_ij
        acc = acc * alpha[:, None]
        v = tl.load(V + base + (start_n + offs_n)[:, None] * HEAD_DIM + offs_d[None, :])
        p = p.to(V.dtype.element_ty)  # fp16, or fp8e5 for the fp8 provider
        acc = tl.dot(p, v, acc)
        m_i = m_ij
    m_i += tl.math.log2(l_i)
    acc = acc / l_i[:, None]
    tl.store(M + off_hz * N_CTX + offs_m, m_i)
    tl.store(Out + base + offs_m[:, None] * HEAD_DIM + offs_d[None, :],
             acc.to(Out.dtype.element_ty))


@triton.jit
def cast_e5m2_kernel(X, Y, n, BLOCK: tl.constexpr):
    offs = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
    x = tl.load(X + offs, mask=offs < n)
    tl.store(Y + offs, x.to(tl.float8e5), mask=offs < n)


def attn_case(rng, name, Z, H, N, D, causal, sm_scale, block, fp8=False):
    std = 1.0 if fp8 else 0.5  # the tutorial's fp8 bench: randn, then .to(float8_e5m2)
    q, k, v = (torch.from_numpy((rng.standard_normal((Z, H, N, D)) * std).astype(np.float16))
               for _ in range(3))
    if fp8:
        q, k, v = (x.to(torch.float8_e5m2) for x in (q, k, v))
    o = torch.empty_like(q)
    M = torch.empty((Z * H, N), dtype=torch.float32)
    BM, BN = block
    attn_fwd_kernel[(N // BM, Z * H)](q, k, v, sm_scale, M, o, N, H, HEAD_DIM=D, BLOCK_M=BM,
                                      BLOCK_N=BN, CAUSAL=causal)
    d = dict(q=bits(q), k=bits(k), v=bits(v), o=bits(o), M=M.numpy(), causal=np.bool_(causal),
             sm_scale=np.float32(sm_scale), block=np.array(block, np.int32))
    np.savez_compressed(os.path.join(HERE, name + ".npz"), **d)
    size = os.path.getsize(os.path.join(HERE, name + ".npz"))
    print(f"{name}: Z={Z} H={H} N_CTX={N} D={D} causal={causal} {size / 1024:.1f} KiB", flush=True)


MX_FMT = {"e4m3": 0, "e5m2": 1, "e2m1": 4}


def run_mx(a, sa, fa, b, sb, fb, *, K, block):
    """Interpreter output (fp32) of tl.dot_scaled's upcast form."""
    M, N = a.shape[0], b.shape[1]
    c = torch.zeros((M, N), dtype=torch.float32)
    BM, BN, BK = block
    grid = (triton.cdiv(M, BM), triton.cdiv(N, BN))
    mx_dot_kernel[grid](torch.from_numpy(a), torch.from_numpy(b), torch.from_numpy(sa),
                        torch.from_numpy(sb), c, M, N, K, BM=BM, BN=BN, BK=BK,
                        FA=MX_FMT[fa], FB=MX_FMT[fb])
    return c.numpy()


def save_mx(name, a, sa, fa, b, sb, fb, c, *, K, block, exact):
    d = dict(a=a, sa=sa, b=b, sb=sb, c=c, a_fmt=fa, b_fmt=fb, K=np.int64(K),
             M=np.int64(a.shape[0]), N=np.int64(b.shape[1]), block=np.array(block, np.int32),
             exact=np.bool_(exact))
    np.savez_compressed(os.path.join(HERE, name + ".npz"), **d)
    size = os.path.getsize(os.path.join(HERE, name + ".npz"))
    print(f"{name}: M={a.shape[0]} N={b.shape[1]} K={K} {fa} x {fb} {size / 1024:.1f} KiB",
          flush=True)


def mx_codes(rng, shape, fmt, exact):
    """Codes of `fmt`; exact: small dyadic magnitudes (NaN / inf codes never)."""
    if fmt == "e2m1":
        return rng.integers(0, 16, size=shape, dtype=np.uint8)
    if fmt == "e4m3":  # exponent field 5..8 (values 2^-2 .. 2^2) or any finite code
        if exact:
            return (rng.integers(0, 2, size=shape) << 7 | rng.integers(5, 9, size=shape) << 3
                    | rng.integers(0, 8, size=shape)).astype(np.uint8)
        c = rng.integers(0, 256, size=shape).astype(np.uint8)
        return np.where((c & 0x7F) == 0x7F, c & 0xF0, c).astype(np.uint8)
    if exact:  # e5m2, exponent field 13..16
        return (rng.integers(0, 2, size=shape) << 7 | rng.integers(13, 17, size=shape) << 2
                | rng.integers(0, 4, size=shape)).astype(np.uint8)
    c = rng.integers(0, 256, size=shape).astype(np.uint8)
    return np.where((c & 0x7C) == 0x7C, c & 0x83, c).astype(np.uint8)


def pack_e2m1(codes, axis):
    """Two e2m1 codes per byte along `axis`, even index in the low nibble."""
    lo = np.take(codes, np.arange(0, codes.shape[axis], 2), axis=axis)
    hi = np.take(codes, np.arange(1, codes.shape[axis], 2), axis=axis)
    return (lo | (hi << 4)).astype(np.uint8)


def mx_case(rng, name, fa, fb, M, N, K, *, exact, block):
    ac = mx_codes(rng, (M, K), fa, exact)
    bc = mx_codes(rng, (K, N), fb, exact)
    lo, hi = (125, 130) if exact else (117, 138)  # exact: sums within fp32's 24 bits
    sa = rng.integers(lo, hi, size=(M, K // 32)).astype(np.uint8)
    sb = rng.integers(lo, hi, size=(N, K // 32)).astype(np.uint8)
    a = pack_e2m1(ac, 1) if fa == "e2m1" else ac
    b = pack_e2m1(bc, 0) if fb == "e2m1" else bc
    c = run_mx(a, sa, fa, b, sb, fb, K=K, block=block)
    save_mx(name, a, sa, fa, b, sb, fb, c, K=K, block=block, exact=exact)


TL_OUT = {"f32": tl.float32, "bf16": tl.bfloat16, "f16": tl.float16, "i32": tl.int32}
TORCH_OUT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16,
             "i32": torch.int32}
FP8 = (torch.float8_e4m3fn, torch.float8_e5m2)
BITS = {torch.float16: np.uint16, torch.bfloat16: np.uint16, torch.float8_e4m3fn: np.uint8,
        torch.float8_e5m2: np.uint8, torch.int8: np.int8, torch.float32: np.float32,
        torch.int32: np.int32}


def bits(t):
    """Raw element bits of a CPU tensor as a numpy array."""
    view = {torch.float16: torch.int16, torch.bfloat16: torch.int16,
            torch.float8_e4m3fn: torch.uint8, torch.float8_e5m2: torch.uint8}.get(t.dtype)
    a = (t.view(view) if view is not None else t).numpy()
    return a.view(BITS[t.dtype])


def run(a, b, *, out, block, epi=EPI_NONE, sa=None, sb=None):
    M, K = a.shape
    N = b.shape[1]
    BM, BN, BK = block
    c = torch.zeros((M, N), dtype=TORCH_OUT[out])
    sa_t = sa if sa is not None else torch.zeros(1)
    sb_t = sb if sb is not None else torch.zeros(1)
    sa_ld = sa.shape[1] if (sa is not None and sa.dim() == 2) else 0
    sb_ld = sb.shape[1] if (sb is not None and sb.dim() == 2) else 0
    grid = (triton.cdiv(M, BM), triton.cdiv(N, BN))
    mask = a.dtype not in FP8
    if not mask:
        assert M % BM == 0 and N % BN == 0 and K % BK == 0, "fp8 fixtures need whole tiles"
    tiled_dot_kernel[grid](a, b, c, sa_t, sb_t, M, N, K, sa_ld, sb_ld, BM=BM, BN=BN, BK=BK,
                           WIDEN=a.dtype == torch.bfloat16, INT_ACC=a.dtype == torch.int8,
                           EPI=epi, OUT=TL_OUT[out], MASK=mask)
    return c


def save(name, a, b, c, *, block, out, epi=EPI_NONE, sa=None, sb=None, exact=False,
         store_inputs=True, seeds=None, tiles=None):
    """Write <name>.npz.  `tiles` keeps only those output tiles (others left out)."""
    d = dict(a_type=str(_tname(a.dtype)), b_type=str(_tname(b.dtype)), c_type=out,
             block=np.array(block, np.int32),
             epi=np.int32(epi), exact=np.bool_(exact), M=np.int64(a.shape[0]),
             N=np.int64(b.shape[1]), K=np.int64(a.shape[1]),
             a_sha256=hashlib.sha256(bits(a).tobytes()).hexdigest(),
             b_sha256=hashlib.sha256(bits(b).tobytes()).hexdigest())
    if store_inputs:
        d["a"], d["b"] = bits(a), bits(b)
    if seeds is not None:
        d["seeds"] = np.array(seeds, np.int64)
    if sa is not None:
        d["sa"], d["sb"] = sa.numpy(), sb.numpy()
    cb = bits(c)
    if tiles is None:
        d["c"] = cb
    else:
        BM, BN, _ = block
        d["tiles"] = np.array(tiles, np.int32)
        d["c_tiles"] = np.stack([cb[i * BM:(i + 1) * BM, j * BN:(j + 1) * BN] for i, j in tiles])
    np.savez_compressed(os.path.join(HERE, name + ".npz"), **d)
    size = os.path.getsize(os.path.join(HERE, name + ".npz"))
    print(f"{name}: M={a.shape[0]} N={b.shape[1]} K={a.shape[1]} block={block} out={out} "
          f"{size / 1024:.1f} KiB", flush=True)


def _tname(dt):
    return {torch.float16: "f16", torch.bfloat16: "bf16", torch.int8: "i8",
            torch.float8_e4m3fn: "f8e4m3", torch.float8_e5m2: "f8e5m2"}[dt]


def dyadic(shape, rng, lim, denom, dtype):
    """Integers in [-lim, lim] over `denom`: exact in the element type."""
    v = rng.integers(-lim, lim + 1, size=shape).astype(np.float32) / np.float32(denom)
    return torch.from_numpy(v).to(dtype)


def normal(shape, rng, scale, dtype):
    v = rng.standard_normal(shape, dtype=np.float32) * np.float32(scale)
    return torch.from_numpy(v).to(dtype)


def main():
    rng = np.random.default_rng(20261201)

    # C1, the reference-sized CPU config: fp16 512^3, BLOCK 64x64x32, fp32 C.
    # Inputs are regenerated from seeds 1 and 2 (numpy PCG64 standard_normal /
    # sqrt(512), rounded to fp16 by numpy); their hashes are stored to prove it.
    K = 512
    a = torch.from_numpy((np.random.default_rng(1).standard_normal((512, K), dtype=np.float32)
                          * np.float32(K ** -0.5)).astype(np.float16))
    b = torch.from_numpy((np.random.default_rng(2).standard_normal((K, 512), dtype=np.float32)
                          * np.float32(K ** -0.5)).astype(np.float16))
    c = run(a, b, out="f32", block=(64, 64, 32))
    save("c1_fp16_512", a, b, c, block=(64, 64, 32), out="f32", store_inputs=False,
         seeds=(1, 2), tiles=[(0, 0), (3, 5), (7, 7)])

    # fp16 -> fp32, edge tiles in M and N and a K tail (40 = 32 + 8): exact.
    a = dyadic((70, 40), rng, 16, 8, torch.float16)
    b = dyadic((40, 56), rng, 16, 8, torch.float16)
    save("fp16_f32_edges_exact", a, b, run(a, b, out="f32", block=(64, 64, 32)),
         block=(64, 64, 32), out="f32", exact=True)

    # fp16 -> fp16 (numpy RNE on the exact fp32 accumulator).
    a = dyadic((48, 64), rng, 16, 8, torch.float16)
    b = dyadic((64, 40), rng, 16, 8, torch.float16)
    save("fp16_f16_rne_exact", a, b, run(a, b, out="f16", block=(32, 32, 32)),
         block=(32, 32, 32), out="f16", exact=True)

    # bf16 -> bf16: tiles widened to fp32, exact accumulator, TRUNCATING cast.
    a = dyadic((48, 72), rng, 255, 16, torch.bfloat16)
    b = dyadic((72, 80), rng, 255, 16, torch.bfloat16)
    save("bf16_bf16_rtz_exact", a, b, run(a, b, out="bf16", block=(32, 64, 32)),
         block=(32, 64, 32), out="bf16", exact=True)

    # bf16 -> fp32 with N(0,1)/sqrt(K) inputs: tolerance (fp32 summation order).
    K = 200
    a = normal((40, K), rng, K ** -0.5, torch.bfloat16)
    b = normal((K, 72), rng, K ** -0.5, torch.bfloat16)
    save("bf16_f32_normal", a, b, run(a, b, out="f32", block=(64, 64, 64)),
         block=(64, 64, 64), out="f32")

    # int8 -> int32, K tail (96 = 64 + 32) and edges: exact.
    a = torch.from_numpy(rng.integers(-127, 128, size=(20, 96), dtype=np.int8))
    b = torch.from_numpy(rng.integers(-127, 128, size=(96, 48), dtype=np.int8))
    save("int8_i32", a, b, run(a, b, out="i32", block=(16, 32, 64)),
         block=(16, 32, 64), out="i32", exact=True)

    # W8A8: bf16((float(acc) * sa[m]) * sb[n]), truncating cast.
    a = torch.from_numpy(rng.integers(-127, 128, size=(5, 128), dtype=np.int8))
    b = torch.from_numpy(rng.integers(-127, 128, size=(128, 64), dtype=np.int8))
    sa = torch.from_numpy(rng.uniform(0.001, 0.02, size=5).astype(np.float32))
    sb = torch.from_numpy(rng.uniform(0.001, 0.02, size=64).astype(np.float32))
    save("w8a8_rowcol_rtz", a, b,
         run(a, b, out="bf16", block=(16, 32, 64), epi=EPI_ROWCOL, sa=sa, sb=sb),
         block=(16, 32, 64), out="bf16", epi=EPI_ROWCOL, sa=sa, sb=sb, exact=True)

    # fp8 e4m3, 128-wide K blocks with fp32 scales: A per 1x128 group, B per
    # 128x128 block.  Values j/8, |j| <= 15 (exact in e4m3; exact partials).
    M, N, K = 16, 256, 256
    a = dyadic((M, K), rng, 15, 8, torch.float8_e4m3fn)
    b = dyadic((K, N), rng, 15, 8, torch.float8_e4m3fn)
    sa = torch.from_numpy(rng.uniform(0.001, 0.01, size=(M, K // 128)).astype(np.float32))
    sb = torch.from_numpy(rng.uniform(0.001, 0.01, size=(K // 128, N // 128)).astype(np.float32))
    save("fp8_block128_f32_exact", a, b,
         run(a, b, out="f32", block=(16, 128, 128), epi=EPI_BLOCK128, sa=sa, sb=sb),
         block=(16, 128, 128), out="f32", epi=EPI_BLOCK128, sa=sa, sb=sb, exact=True)

    # fp8 e4m3 with N(0,1) values quantised by per-group amax/448 scales, the
    # C5 recipe, at a small size; bf16 output (truncating cast): tolerance.
    M, N, K = 32, 128, 256
    x = rng.standard_normal((M, K), dtype=np.float32)
    y = rng.standard_normal((K, N), dtype=np.float32)
    sa_np = np.abs(x.reshape(M, K // 128, 128)).max(axis=2) / np.float32(448)
    sb_np = np.abs(y.reshape(K // 128, 128, N // 128, 128)).max(axis=(1, 3)) / np.float32(448)
    qa = torch.from_numpy(x / np.repeat(sa_np, 128, axis=1)).to(torch.float8_e4m3fn)
    qb = torch.from_numpy(y / np.repeat(np.repeat(sb_np, 128, axis=0), 128, axis=1)
                          ).to(torch.float8_e4m3fn)
    sa, sb = torch.from_numpy(sa_np.astype(np.float32)), torch.from_numpy(sb_np.astype(np.float32))
    save("fp8_block128_bf16_normal", qa, qb,
         run(qa, qb, out="bf16", block=(32, 128, 128), epi=EPI_BLOCK128, sa=sa, sb=sb),
         block=(32, 128, 128), out="bf16", epi=EPI_BLOCK128, sa=sa, sb=sb)

    # tl.dot_scaled (MX), fp32 C.  Exact: every term and partial sum fits
    # fp32, so any summation order gives these bits.  Edges in M and N and a
    # K that is not a multiple of the GPU's 128 (fp8) / 256 (fp4) step.
    mx_case(rng, "mx_e4m3_e5m2_f32_exact", "e4m3", "e5m2", 40, 48, 96, exact=True,
            block=(32, 32, 32))
    mx_case(rng, "mx_e2m1_f32_exact", "e2m1", "e2m1", 24, 32, 160, exact=True,
            block=(16, 32, 32))
    mx_case(rng, "mx_e5m2_e4m3_f32_exact", "e5m2", "e4m3", 16, 64, 288, exact=True,
            block=(16, 32, 64))
    # full-range codes and scales 2^-10 .. 2^10: tolerance (fp32 summation order)
    mx_case(rng, "mx_e4m3_f32_random", "e4m3", "e4m3", 32, 64, 256, exact=False,
            block=(32, 32, 64))
    mx_case(rng, "mx_e2m1_f32_random", "e2m1", "e2m1", 32, 48, 512, exact=False,
            block=(32, 16, 64))

    # fused attention forward (the tutorial's test_op recipe, smaller): causal
    # with the LoopSplit on-band branch, and plain
    attn_case(rng, "attn_fwd_causal", 1, 2, 256, 64, True, 0.5, (64, 32))
    attn_case(rng, "attn_fwd_plain", 2, 1, 128, 64, False, 1.3, (64, 32))

    # fp8 tt.dot with e5m2 operands (the tutorial's p . v with fp8e5 p,
    # R:pass/LoopSplit/06-fused-attention.py:81-85), fp32 C.  Exact: small
    # dyadic values (also exact in the MFMA's fixed-point group sums).
    a = dyadic((256, 256), rng, 7, 4, torch.float8_e5m2)
    b = dyadic((256, 256), rng, 7, 4, torch.float8_e5m2)
    save("fp8e5_f32_exact", a, b, run(a, b, out="f32", block=(64, 64, 64)),
         block=(64, 64, 64), out="f32", exact=True)
    a = dyadic((128, 384), rng, 15, 8, torch.float8_e4m3fn)
    b = dyadic((384, 256), rng, 7, 4, torch.float8_e5m2)
    save("fp8e4e5_f32_exact", a, b, run(a, b, out="f32", block=(64, 64, 64)),
         block=(64, 64, 64), out="f32", exact=True)
    a = normal((64, 256), rng, 1.0, torch.float8_e5m2)
    b = normal((256, 128), rng, 1.0, torch.float8_e5m2)
    save("fp8e5_f32_normal", a, b, run(a, b, out="f32", block=(64, 64, 64)),
         block=(64, 64, 64), out="f32")

    fp8_attention(np.random.default_rng(20261202))


def e5m2_cast_inputs(rng):
    """fp32 values for the interpreter's fp32 -> e5m2 cast: every binade from
    fp32 subnormals to past e5m2's largest finite, with significands that hit
    the round bit, ties, sticky bits and the carry out of the top 2 bits."""
    sigs = [0, 1, 1 << 19, 1 << 20, (1 << 20) | 1, 1 << 21, (1 << 21) | (1 << 20), 2 << 21,
            3 << 21, (3 << 21) | (1 << 20), (3 << 21) | (1 << 20) | 1, (2 << 21) | (1 << 20),
            0x7FFFFF]
    bits = []
    for e in list(range(0, 8)) + list(range(90, 146)):
        for m in sigs + [int(x) for x in rng.integers(0, 1 << 23, size=4)]:
            bits.append((e << 23) | m)
    bits = np.array(bits, dtype=np.uint32)
    bits = np.concatenate([bits, bits | np.uint32(0x80000000)])
    return bits.view(np.float32)


def fp8_attention(rng):
    """The tutorial's fp8 forward (R:pass/LoopSplit/06-fused-attention.py
    :774-779 bench inputs, :81-82 p.to(fp8e5), :238 o in q's type): e5m2 q, k,
    v, p and o; and the fp32 -> e5m2 cast it applies to p and o."""
    x = e5m2_cast_inputs(rng)
    y = torch.empty(x.size, dtype=torch.float8_e5m2)
    cast_e5m2_kernel[(triton.cdiv(x.size, 256),)](torch.from_numpy(x), y, x.size, BLOCK=256)
    np.savez_compressed(os.path.join(HERE, "e5m2_cast_interp.npz"), x=x,
                        y=y.view(torch.uint8).numpy())
    print(f"e5m2_cast_interp: {x.size} values", flush=True)
    attn_case(rng, "attn_fwd_fp8_causal", 1, 2, 256, 64, True, 1.3, (64, 32), fp8=True)
    attn_case(rng, "attn_fwd_fp8_plain", 1, 1, 128, 64, False, 0.5, (64, 32), fp8=True)


def e4m3_max_codes(rng):
    """e4m3 codes 0x7F / 0xFF (S.1111.111) inside a tiled fp8 dot.  OCP e4m3fn
    (Triton's fp8e4nv) makes them NaN; the interpreter's generic converter
    (T:runtime/interpreter.py:202-263) decodes them as +-480.  Dyadic values
    elsewhere (j/8, |j| <= 15), so every partial sum is exact in fp32 and the
    fixture pins the interpreter's decode bit for bit.  Max codes sit in A
    rows 3, 17 and 40 and in B column 9."""
    M, N, K = 64, 64, 128
    a = bits(dyadic((M, K), rng, 15, 8, torch.float8_e4m3fn)).copy()
    b = bits(dyadic((K, N), rng, 15, 8, torch.float8_e4m3fn)).copy()
    a[3, 5], a[17, 77], a[40, 127] = 0x7F, 0xFF, 0x7F
    b[100, 9] = 0xFF
    at = torch.from_numpy(a).view(torch.float8_e4m3fn)
    bt = torch.from_numpy(b).view(torch.float8_e4m3fn)
    save("fp8e4m3_maxcode_f32_exact", at, bt, run(at, bt, out="f32", block=(32, 32, 64)),
         block=(32, 32, 64), out="f32", exact=True)


if __name__ == "__main__":
    if not os.environ.get("TRITON_INTERPRET"):
        sys.exit("set TRITON_INTERPRET=1")
    if sys.argv[1:] == ["e4m3_max_codes"]:  # only this fixture
        e4m3_max_codes(np.random.default_rng(20261203))
    else:
        main()
        e4m3_max_codes(np.random.default_rng(20261203))
