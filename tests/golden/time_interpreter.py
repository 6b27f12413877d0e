"""Time the reference's CPU execution of the tiled dot -- the Triton
interpreter (TRITON_INTERPRET=1) running make_golden.py's tiled_dot_kernel --
on BASELINE's configs, in the build container:

    python tests/golden/time_interpreter.py

C1 runs in full.  C2-C5 run one program (one output tile over the whole K) and
are extrapolated by the program count: programs are independent and run one
after another (T:runtime/interpreter.py:1353-1357).  tl.dot is numpy matmul,
so the BLAS thread count matters and is printed.  Needs the third-party
triton package; nothing on the GPU box runs this.
"""
import os
import sys
import time

os.environ["TRITON_INTERPRET"] = "1"
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

import numpy as np  # noqa: E402
import torch  # noqa: E402

import make_golden as mg  # noqa: E402


def timed(fn, reps=2):
    best = float("inf")
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        best = min(best, time.perf_counter() - t0)
    return best


def main():
    rng = np.random.default_rng(0)
    normal = lambda shape, s, dt: torch.from_numpy(
        (rng.standard_normal(shape) * s).astype(np.float32)).to(dt)
    rows = []

    # C1: fp16 512^3, BLOCK 64x64x32, fp32 C -- the whole grid
    a, b = normal((512, 512), 512 ** -0.5, torch.float16), normal((512, 512), 512 ** -0.5,
                                                                  torch.float16)
    t = timed(lambda: mg.run(a, b, out="f32", block=(64, 64, 32)))
    rows.append(("C1 fp16 512^3, BLOCK 64x64x32, fp32 C (full grid)", t, 1, 2 * 512 ** 3))

    # C2 / C3: bf16, one 256x256 program over K, x 256 programs
    for K, name in ((4096, "C2 bf16 4096^3"), (4000, "C3 bf16 4096x4096x4000")):
        a, b = normal((256, K), K ** -0.5, torch.bfloat16), normal((K, 256), K ** -0.5,
                                                                   torch.bfloat16)
        t = timed(lambda: mg.run(a, b, out="bf16", block=(256, 256, 64)))
        rows.append((f"{name}, 256x256x64 programs, bf16 C", t, 256, 2 * 4096 * 4096 * K))

    # C4: W8A8 M=16, N=K=8192: one 16x128 program over K, x 64
    a = torch.from_numpy(rng.integers(-127, 128, size=(16, 8192), dtype=np.int8))
    b = torch.from_numpy(rng.integers(-127, 128, size=(8192, 128), dtype=np.int8))
    sa = torch.from_numpy(rng.uniform(0.001, 0.02, 16).astype(np.float32))
    sb = torch.from_numpy(rng.uniform(0.001, 0.02, 128).astype(np.float32))
    t = timed(lambda: mg.run(a, b, out="bf16", block=(16, 128, 64), epi=mg.EPI_ROWCOL,
                             sa=sa, sb=sb))
    rows.append(("C4 W8A8 M=16 N=K=8192, 16x128x64 programs", t, 64, 2 * 16 * 8192 * 8192))

    # C5: fp8 e4m3 block-scaled 2048x7168x7168: one 128x128 program over K, x 896
    K = 7168
    a = normal((128, K), 1.0, torch.float8_e4m3fn)
    b = normal((K, 128), 1.0, torch.float8_e4m3fn)
    sa = torch.from_numpy(rng.uniform(0.001, 0.01, (128, K // 128)).astype(np.float32))
    sb = torch.from_numpy(rng.uniform(0.001, 0.01, (K // 128, 1)).astype(np.float32))
    t = timed(lambda: mg.run(a, b, out="bf16", block=(128, 128, 128), epi=mg.EPI_BLOCK128,
                             sa=sa, sb=sb), reps=1)
    rows.append(("C5 fp8 block-scaled 2048x7168x7168, 128x128x128 programs", t,
                 (2048 // 128) * (7168 // 128), 2 * 2048 * 7168 * 7168))

    env = {k: os.environ.get(k, "unset") for k in ("OMP_NUM_THREADS", "OPENBLAS_NUM_THREADS")}
    print(f"cores: {os.cpu_count()}, {env}, numpy {np.__version__}")
    print("| config | one run (s) | programs | extrapolated (s) | GFLOP/s |")
    print("|---|---|---|---|---|")
    for name, t, n, flops in rows:
        total = t * n
        print(f"| {name} | {t:.3f} | {n} | {total:.1f} | {flops / total / 1e9:.2f} |")


if __name__ == "__main__":
    main()
