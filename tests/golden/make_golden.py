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


TL_OUT = {"f32": tl.float32, "bf16": tl.bfloat16, "f16": tl.float16, "i32": tl.int32}
TORCH_OUT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16,
             "i32": torch.int32}
TORCH_IN = {"f16": torch.float16, "bf16": torch.bfloat16, "i8": torch.int8,
            "f8e4m3": torch.float8_e4m3fn}
BITS = {torch.float16: np.uint16, torch.bfloat16: np.uint16, torch.float8_e4m3fn: np.uint8,
        torch.int8: np.int8, torch.float32: np.float32, torch.int32: np.int32}


def bits(t):
    """Raw element bits of a CPU tensor as a numpy array."""
    view = {torch.float16: torch.int16, torch.bfloat16: torch.int16,
            torch.float8_e4m3fn: torch.uint8}.get(t.dtype)
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
    mask = a.dtype != torch.float8_e4m3fn
    if not mask:
        assert M % BM == 0 and N % BN == 0 and K % BK == 0, "fp8 fixtures need whole tiles"
    tiled_dot_kernel[grid](a, b, c, sa_t, sb_t, M, N, K, sa_ld, sb_ld, BM=BM, BN=BN, BK=BK,
                           WIDEN=a.dtype == torch.bfloat16, INT_ACC=a.dtype == torch.int8,
                           EPI=epi, OUT=TL_OUT[out], MASK=mask)
    return c


def save(name, a, b, c, *, block, out, epi=EPI_NONE, sa=None, sb=None, exact=False,
         store_inputs=True, seeds=None, tiles=None):
    """Write <name>.npz.  `tiles` keeps only those output tiles (others left out)."""
    d = dict(a_type=str(_tname(a.dtype)), c_type=out, block=np.array(block, np.int32),
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
            torch.float8_e4m3fn: "f8e4m3"}[dt]


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


if __name__ == "__main__":
    if not os.environ.get("TRITON_INTERPRET"):
        sys.exit("set TRITON_INTERPRET=1")
    main()
