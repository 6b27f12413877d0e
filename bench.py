"""Benchmark: tiled tt.dot on one MI355X through the tx_dot C-ABI.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only NAME]

A step is one dot over synthetic inputs already resident in HBM.  The
headline workload is BASELINE configs[1]: bf16 C = A @ B, M = N = K = 4096,
fp32 accumulation, entries N(0,1)/sqrt(K).  `value` is its TFLOP/s (2*M*N*K
per step over the timed region, HIP events on the launch stream).  The other
configs are reported under "secondary": the LoopSplit K-tail and edge cases,
int8 W8A8 decode (M = 1, 16, 64, 256; HBM-bound, each launch after a
512 MiB read that flushes the 256 MB MALL so B streams from HBM: `ms` is a
launch inside the stream, (flush, launch) sequences minus the flushes alone;
`ms_isolated` a lone launch between its own events), the fp8
block-scaled dot, tl.dot_scaled's MX formats (mxfp8 e4m3 and mxfp4 e2m1
with e8m0 scales per 32 K, fp32 C), and the fused attention forward of the
reference's tutorial at its benchmark shape (BATCH 4, 32 heads, HEAD_DIM 64).

cpu_baseline: the CPU oracle (a C restatement of the Triton interpreter's
tiled dot, oracle/) on the host cores for the same bf16 4096^3 inputs; it
also checks the GPU output of the timed run against that result.
"""
import argparse
import ctypes
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "triton-ext_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "tt.dot TFLOP/s + % MFMA/HBM roofline (bf16 4096^3; int8 W8A8 M=16)"
PEAK_BF16 = 2516.6e12
PEAK_I8 = 5033.2e12
PEAK_F4 = 10066.4e12
HBM = 8.0e12
# HBM bytes per launch of the bf16 4096^3 kernel: rocprofv3 FETCH_SIZE + WRITE_SIZE of one
# dispatch, each scaled by the counter's reading for a 256 MiB copy (--copy-probe): FETCH x2.0,
# WRITE x1.0 (profiles/gemm16_bf16_4096.md).
TRAFFIC_BF16_4096 = 235.2e6
# The same for the W8A8 M=16 decode kernel (profiles/decode_i8_w8a8_m16.md).
TRAFFIC_W8A8_M16 = 72.4e6


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", default="",
                    help="secondary workloads to run, comma-separated: ceiling, phases (where a "
                         "headline launch's time goes), tiles, c1, vendor (vendor8: hipBLASLt's 8-bit GEMMs "
                         "only; vendor_decode: its decode shapes only), tail, "
                         "w8a8 (or "
                         "w8a8_1, w8a8_16, w8a8_64, w8a8_256; w8a8 also runs i32_16, the unscaled "
                         "int8 -> int32 decode at M=16, and i32_16_kmajor, the same with B "
                         "K-major), w8a8_kmajor (or w8a8_kmajor_1, _16, _64, _256: W8A8 with the "
                         "weight kept [N][K]), bf16_decode (or bf16_decode_1, _16, _64, _96: "
                         "bf16 at N = K = 8192 on the 16-bit decode kernel; bf16_decode_kmajor, "
                         "or _1, _16, _64, _96: the same with B K-major), decode16_widths (not in the "
                         "default run: bf16 with strips of 64 and of 128 columns, M = 16 .. 80 and a sweep "
                         "of N and K at M = 64 and 16), mid_m (or mid_m_bf16_128, _256, "
                         "_512, mid_m_fp8_256: a few hundred rows on the split-K tiles), fp8_decode (or "
                         "fp8_decode_1, _16, _64: block-scaled e4m3 at N = K = 7168 on the fp8 "
                         "decode kernel), int8, fp8 (fp8u: the unscaled 4096^3 line only), kmajor (bf16 "
                         "4096^3, int8 and fp8 4096^3 with B K-major), "
                         "mx (or mxfp8, mxfp4, "
                         "mxfp8_4096, mxfp8_8192, mxfp4_4096, mxfp4_8192), mxbf16 (or mxbf16_fp4, mxbf16_fp8: "
                         "bf16 x MX), attn (or attn_1024, attn_4096, "
                         "attn_16384; attn_fp8 or attn_fp8_<N> for e5m2; attn_d128 for head dim 128; "
                         "attn_vendor adds torch sdpa beside each) "
                         "(default: all); "
                         "the bf16 "
                         "headline always runs")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only copy 256 MiB five times (a transfer of known size that scales the "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE counters), then exit")
    return ap.parse_args()


class Launcher:
    """Plan once, then launch through tx_dot_launch with minimal host work."""

    def __init__(self, tx, a, b, out, sa=None, sb=None, scale_mode=None, block=(0, 0, 0)):
        import torch
        self.tx = tx
        self.L = tx.load()
        sm = scale_mode if scale_mode is not None else tx.SCALE_NONE
        self.plan = tx.plan_for(a, b, tx.tx_type(out), sm, block)
        stream = torch.cuda.current_stream().cuda_stream
        self.ws = tx.workspace_for(self.plan, a.device, stream)
        self.args = (ctypes.byref(self.plan), a.data_ptr(), b.data_ptr(), out.data_ptr(),
                     None if sa is None else sa.data_ptr(), None if sb is None else sb.data_ptr(),
                     None if self.ws is None else self.ws.data_ptr(),
                     0 if self.ws is None else self.ws.numel(), stream)
        self.keep = (a, b, out, sa, sb)

    def __call__(self):
        rc = self.L.tx_dot_launch(*self.args)
        if rc != 0:
            raise RuntimeError(self.L.tx_get_last_error().decode())


def plan_info(tx, p, **extra):
    """What the planning passes chose for a line: kernel, tile and the
    arith_intensity pass's FLOP/byte and bound."""
    return dict(kernel=tx.load().tx_kernel_name(p.kernel).decode(),
                tile=[p.desc.block_m, p.desc.block_n, p.desc.block_k],
                intensity=round(p.intensity, 1),
                bound="mfma" if p.bound == tx.BOUND_MFMA else "hbm", **extra)


MIN_WARMUP_S = 0.1


def warm(fn, warmup):
    """`warmup` untimed launches, then more until at least MIN_WARMUP_S of GPU work has run:
    MI355X's clocks take tens of milliseconds to settle under MFMA load (triton's do_bench
    warms up by time for the same reason)."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < MIN_WARMUP_S:
        for _ in range(20):
            fn()
        torch.cuda.synchronize()


def time_back_to_back(fn, steps, warmup):
    """Average ms per launch over `steps` back-to-back launches (events on the launch stream)."""
    import torch
    warm(fn, warmup)
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(steps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / steps


def time_cold(fn, steps, warmup, flush):
    """Median ms of single launches, each bracketed by events, with `flush` run before each."""
    import torch
    warm(fn, warmup)
    times = []
    for _ in range(steps):
        flush()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        fn()
        e.record()
        times.append((s, e))
    torch.cuda.synchronize()
    ms = sorted(s.elapsed_time(e) for s, e in times)
    return ms[len(ms) // 2], ms


def time_cold_in_stream(fn, flush, reps=30, rounds=5):
    """Per-launch ms of a cold launch inside a stream: (flush, fn) x reps minus
    flush x reps, each sequence bracketed by events, median over rounds.  The
    launch follows another kernel, as in a decode loop, so its dispatch
    overlaps that kernel's tail; the difference is the launch's own time."""
    import torch
    out = []
    for _ in range(rounds):
        torch.cuda.synchronize()
        s0, e0 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s1, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record()
        for _ in range(reps):
            flush()
            fn()
        e0.record()
        s1.record()
        for _ in range(reps):
            flush()
        e1.record()
        torch.cuda.synchronize()
        out.append((s0.elapsed_time(e0) - s1.elapsed_time(e1)) / reps)
    return sorted(out)[len(out) // 2]


def make_flush(dev):
    """Read 512 MiB (2x the 256 MB MALL) so the next kernel's operands come from HBM.

    A read, not a write: a write-flush would leave the caches full of dirty
    lines whose write-back then competes with the timed kernel's reads."""
    import torch
    buf = torch.ones((512 << 20) // 4, dtype=torch.float32, device=dev)

    def flush():
        buf.sum()
    return flush


def bf16_inputs(M, N, K, dev, seed):
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    a = (torch.randn((M, K), generator=g, device=dev, dtype=torch.float32) / math.sqrt(K)).to(torch.bfloat16)
    b = (torch.randn((K, N), generator=g, device=dev, dtype=torch.float32) / math.sqrt(K)).to(torch.bfloat16)
    return a, b


def bench_bf16(tx, dev, M, N, K, steps, warmup, seed=1):
    import torch
    a, b = bf16_inputs(M, N, K, dev, seed)
    c = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    run = Launcher(tx, a, b, c)
    ms = time_back_to_back(run, steps, warmup)
    flops = 2.0 * M * N * K
    p = run.plan
    return dict(workload=f"bf16 {M}x{N}x{K}", ms=ms, tflops=flops / ms / 1e9,
                frac=flops / ms / 1e-3 / PEAK_BF16,
                plan=plan_info(tx, p, k_split=p.k_split, k_main_steps=p.k_main_steps,
                               k_tail=p.k_tail, m_edge=p.m_edge, n_edge=p.n_edge,
                               group_m=p.group_m)), (a, b, c)


def bench_c1(tx, dev, steps, warmup, seed=1):
    """BASELINE configs[0], the reference's CPU-runnable case: fp16 512^3 with
    BLOCK 64x64x32 and fp32 C (a latency-bound launch: 64 small tiles)."""
    import torch
    M = N = K = 512
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    a = (torch.randn((M, K), generator=g, device=dev) / math.sqrt(K)).to(torch.float16)
    b = (torch.randn((K, N), generator=g, device=dev) / math.sqrt(K)).to(torch.float16)
    c = torch.empty((M, N), dtype=torch.float32, device=dev)
    run = Launcher(tx, a, b, c, block=(64, 64, 32))
    ms = time_back_to_back(run, max(steps, 200), warmup)
    flops = 2.0 * M * N * K
    return dict(workload="fp16 512x512x512, BLOCK 64x64x32, fp32 C (BASELINE configs[0])", ms=ms,
                tflops=flops / ms / 1e9, frac=flops / ms / 1e-3 / PEAK_BF16,
                plan=plan_info(tx, run.plan, grid=run.plan.grid_x))


def bench_bf16_kmajor(tx, dev, M, N, K, steps, warmup, seed=1):
    """The same dot with B stored K-major ([N, K] row-major, passed as its transpose):
    the q @ k.T layout of attention."""
    import torch
    a, b = bf16_inputs(M, N, K, dev, seed)
    bt = b.t().contiguous().t()   # same values, K-major storage
    c = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    run = Launcher(tx, a, bt, c)
    ms = time_back_to_back(run, steps, warmup)
    flops = 2.0 * M * N * K
    return dict(workload=f"bf16 {M}x{N}x{K}, B K-major (q @ k.T)", ms=ms, tflops=flops / ms / 1e9,
                frac=flops / ms / 1e-3 / PEAK_BF16, plan=plan_info(tx, run.plan))


def bench_8bit_kmajor(tx, dev, kind, M, N, K, steps, warmup, seed=1):
    """int8 -> int32 or unscaled fp8 e4m3 -> fp32 with B stored K-major ([N, K] row-major,
    passed as its transpose), on the 256x256x128 tile."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    if kind == "int8":
        a = torch.randint(-127, 128, (M, K), generator=g, device=dev, dtype=torch.int8)
        k = torch.randint(-127, 128, (N, K), generator=g, device=dev, dtype=torch.int8)
        c = torch.empty((M, N), dtype=torch.int32, device=dev)
        what = f"int8 {M}x{N}x{K}, int32 C"
    else:
        a = torch.randn((M, K), generator=g, device=dev).to(torch.float8_e4m3fn)
        k = torch.randn((N, K), generator=g, device=dev).to(torch.float8_e4m3fn)
        c = torch.empty((M, N), dtype=torch.float32, device=dev)
        what = f"fp8 e4m3 {M}x{N}x{K}, fp32 C"
    run = Launcher(tx, a, k.t(), c)
    assert run.plan.desc.flags & tx.FLAG_B_KMAJOR
    ms = time_back_to_back(run, steps, warmup)
    ops = 2.0 * M * N * K
    return dict(workload=f"{what}, B K-major (q @ k.T)", ms=ms, tops=ops / ms / 1e9,
                frac=ops / ms / 1e-3 / PEAK_I8, plan=plan_info(tx, run.plan))


def bench_vendor_bf16(dev, M, N, K, steps, warmup, seed=1):
    """hipBLASLt (torch.matmul) on the same workload and timing: a reference point only."""
    import torch
    a, b = bf16_inputs(M, N, K, dev, seed)
    c = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    ms = time_back_to_back(lambda: torch.matmul(a, b, out=c), steps, warmup)
    return dict(workload=f"hipBLASLt (torch.matmul) bf16 {M}x{N}x{K}", ms=ms,
                tflops=2.0 * M * N * K / ms / 1e9)


def bench_vendor_8bit(dev, steps, warmup, seed=1):
    """hipBLASLt's 8-bit GEMMs at 4096^3, a reference point only: torch._scaled_mm on
    e4m3 (B K-contiguous, as it requires; one tensor-wide scale) with fp32 C -- the type
    an fp8 x fp8 tt.dot yields -- and with bf16 C, and torch._int_mm (int32 C)."""
    import torch
    M = N = K = 4096
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    a = torch.randn((M, K), generator=g, device=dev).to(torch.float8_e4m3fn)
    bt = torch.randn((N, K), generator=g, device=dev).to(torch.float8_e4m3fn)
    ai = torch.randint(-127, 128, (M, K), generator=g, device=dev, dtype=torch.int8)
    bi = torch.randint(-127, 128, (K, N), generator=g, device=dev, dtype=torch.int8)
    one = torch.ones((), device=dev)
    out = []
    for name, fn in (
            ("fp8 e4m3, fp32 C", lambda: torch._scaled_mm(a, bt.t(), scale_a=one, scale_b=one,
                                                           out_dtype=torch.float32)),
            ("fp8 e4m3, bf16 C", lambda: torch._scaled_mm(a, bt.t(), scale_a=one, scale_b=one,
                                                           out_dtype=torch.bfloat16)),
            ("int8, int32 C", lambda: torch._int_mm(ai, bi))):
        try:
            ms = time_back_to_back(fn, steps, warmup)
        except Exception as e:  # a torch build without the op: no vendor line, no failure
            print(f"# hipBLASLt {name}: not available ({type(e).__name__})", file=sys.stderr)
            continue
        out.append(dict(workload=f"hipBLASLt {name} {M}x{N}x{K}", ms=ms,
                        tflops=2.0 * M * N * K / ms / 1e9))
    return out


def bench_w8a8(tx, dev, M, N, K, steps, warmup, flush, seed=3, block=(0, 0, 0), kmajor=False):
    """W8A8 of decode shape, B row-major (config 3); kmajor: the weight kept [N][K] and
    passed as its transpose."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    a = torch.randint(-127, 128, (M, K), generator=g, device=dev, dtype=torch.int8)
    b = torch.randint(-127, 128, (K, N), generator=g, device=dev, dtype=torch.int8)
    if kmajor:
        b = b.t().contiguous().t()   # same values, K-major storage
    sa = torch.rand((M,), generator=g, device=dev) * 0.019 + 0.001
    sb = torch.rand((N,), generator=g, device=dev) * 0.019 + 0.001
    c = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    run = Launcher(tx, a, b, c, sa, sb, tx.SCALE_ROWCOL, block)
    assert bool(run.plan.desc.flags & tx.FLAG_B_KMAJOR) == kmajor
    iso, _ = time_cold(run, steps, warmup, flush)
    med = time_cold_in_stream(run, flush)
    warm = time_back_to_back(run, steps, warmup)
    nbytes = M * K + K * N + M * N * 2 + 4 * (M + N)
    p = run.plan
    # ms: a cold launch (B from HBM) inside a stream; ms_isolated: a lone launch
    # bracketed by its own events (adds the dispatch latency a stream hides)
    return dict(workload=f"int8 W8A8 M={M} N={N} K={K}" + (", B K-major" if kmajor else ""),
                ms=med, ms_isolated=iso,
                ms_warm_mall=warm, gbps=nbytes / med / 1e6, frac_hbm=nbytes / med / 1e-3 / HBM,
                tops=2.0 * M * N * K / med / 1e9,
                plan=plan_info(tx, p, split_k=p.split_k, grid=p.grid_x))


def bench_decode_i32(tx, dev, M, N, K, steps, warmup, flush, seed=3, kmajor=False):
    """int8 x int8 -> int32 tt.dot of decode shape (no scales): the W8A8 decode kernel with
    its int32 epilogue, timed like the W8A8 lines (cold, B from HBM).  kmajor: B stored
    [N][K] and passed as its transpose (the 8-bit decode kernel's int8 form)."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    a = torch.randint(-127, 128, (M, K), generator=g, device=dev, dtype=torch.int8)
    b = torch.randint(-127, 128, (K, N), generator=g, device=dev, dtype=torch.int8)
    if kmajor:
        b = b.t().contiguous().t()   # same values, K-major storage
    c = torch.empty((M, N), dtype=torch.int32, device=dev)
    run = Launcher(tx, a, b, c)
    assert bool(run.plan.desc.flags & tx.FLAG_B_KMAJOR) == kmajor
    iso, _ = time_cold(run, steps, warmup, flush)
    med = time_cold_in_stream(run, flush)
    nbytes = M * K + K * N + M * N * 4
    p = run.plan
    return dict(workload=f"int8 -> int32 (no scales) M={M} N={N} K={K}" +
                (", B K-major" if kmajor else ""), ms=med, ms_isolated=iso,
                gbps=nbytes / med / 1e6, frac_hbm=nbytes / med / 1e-3 / HBM,
                tops=2.0 * M * N * K / med / 1e9,
                plan=plan_info(tx, p, split_k=p.split_k, grid=p.grid_x))


def bench_decode16(tx, dev, M, N, K, steps, warmup, flush, seed=3, kmajor=False):
    """bf16 x bf16 -> bf16 tt.dot of decode shape: the 16-bit decode kernel (B streamed
    once), timed like the W8A8 lines (cold, B from HBM); algorithmic bytes A, B and C once.
    kmajor: B stored [N][K] and passed as its transpose (q @ k.T; a weight kept [out][in])."""
    import torch
    a, b = bf16_inputs(M, N, K, dev, seed)
    if kmajor:
        b = b.t().contiguous().t()   # same values, K-major storage
    c = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    run = Launcher(tx, a, b, c)
    assert bool(run.plan.desc.flags & tx.FLAG_B_KMAJOR) == kmajor
    iso, _ = time_cold(run, steps, warmup, flush)
    med = time_cold_in_stream(run, flush)
    warm = time_back_to_back(run, steps, warmup)
    nbytes = 2 * (M * K + K * N + M * N)
    p = run.plan
    return dict(workload=f"bf16 decode M={M} N={N} K={K}" + (", B K-major" if kmajor else ""),
                ms=med, ms_isolated=iso,
                ms_warm_mall=warm, gbps=nbytes / med / 1e6, frac_hbm=nbytes / med / 1e-3 / HBM,
                tflops=2.0 * M * N * K / med / 1e9,
                plan=plan_info(tx, p, split_k=p.split_k, grid=p.grid_x))


def bench_mid_m(tx, dev, kind, M, N, K, flush, seed=7):
    """Dots of a few hundred rows (a batch past the decode kernels), cold in a stream: the
    256x256 tiles with split-K (kind "bf16": bf16 C; "fp8": e4m3 with 128-block scales, bf16
    C), beside hipBLASLt's bf16 (torch.matmul) on the same shapes and timing."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    c = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    if kind == "bf16":
        a, b = bf16_inputs(M, N, K, dev, seed)
        run = Launcher(tx, a, b, c)
        vendor = time_cold_in_stream(lambda: torch.matmul(a, b, out=c), flush)
        what = f"bf16 M={M} N={N} K={K}"
    else:
        qa, qb, sa, sb = fp8_block_inputs_dev(M, N, K, dev, seed)
        run = Launcher(tx, qa, qb, c, sa, sb, tx.SCALE_BLOCK128)
        vendor = None
        what = f"fp8 e4m3 block-scaled M={M} N={N} K={K}"
    ms = time_cold_in_stream(run, flush)
    p = run.plan
    return dict(workload=what + ", split-K", ms=ms, tflops=2.0 * M * N * K / ms / 1e9,
                ms_vendor=vendor,
                plan=plan_info(tx, p, split_k=p.split_k, grid=[p.grid_x, p.grid_y]))


def bench_decode16_widths(tx, dev, flush, seed=7):
    """The 16-bit decode kernel with strips of 64 and of 128 columns named by explicit block,
    bf16, cold in a stream: N = K = 8192 at M = 16 .. 80 with B row-major and K-major, then
    M = 64 over B from 2^23 to 2^28 elements (B row-major), then M = 16 at N = 8192 .. 28672."""
    import torch
    out = []
    cases = [(M, 8192, 8192, km) for km in (False, True) for M in (16, 32, 48, 64, 80)]
    cases += [(64, n, k, False) for n, k in ((1024, 8192), (2048, 8192), (4096, 4096),
                                             (8192, 2048), (4096, 8192), (16384, 8192),
                                             (28672, 8192))]
    cases += [(16, n, k, km) for n, k in ((8192, 8192), (16384, 4096), (28672, 8192))
              for km in (False, True)]
    for M, N, K, kmajor in cases:
        a, b = bf16_inputs(M, N, K, dev, seed)
        if kmajor:
            b = b.t().contiguous().t()
        c = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        sr = 16 * -(-M // 16)
        ms = {}
        for w in (64, 128):
            run = Launcher(tx, a, b, c, block=(sr, w, 128))
            ms[w] = time_cold_in_stream(run, flush)
        out.append(dict(workload=f"bf16 decode M={M} N={N} K={K}"
                        + (", B K-major" if kmajor else "") + ", strips of 64 / 128 columns",
                        ms_w64=ms[64], ms_w128=ms[128]))
    return out


def fp8_block_inputs_dev(M, N, K, dev, seed):
    """C5's inputs on the device: N(0,1) values quantised to e4m3 per 1 x 128 group of A and
    128 x 128 block of B, fp32 scales."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    a = torch.randn((M, K), generator=g, device=dev)
    b = torch.randn((K, N), generator=g, device=dev)
    kb, nb = (K + 127) // 128, (N + 127) // 128
    sa = a.view(M, kb, 128).abs().amax(dim=2) / 448.0
    sb = b.view(kb, 128, nb, 128).abs().amax(dim=(1, 3)) / 448.0
    qa = (a.view(M, kb, 128) / sa[:, :, None]).view(M, K).to(torch.float8_e4m3fn)
    qb = (b.view(kb, 128, nb, 128) / sb[:, None, :, None]).view(K, N).to(torch.float8_e4m3fn)
    return qa, qb, sa.contiguous(), sb.contiguous()


def bench_decode_f8(tx, dev, M, N, K, steps, warmup, flush, seed=5):
    """fp8 e4m3 block-scaled dot of decode shape (C5's form at small M): the fp8 decode
    kernel, timed like the W8A8 lines (cold, B from HBM); algorithmic bytes A, B, the scales
    and C (bf16) once."""
    import torch
    qa, qb, sa, sb = fp8_block_inputs_dev(M, N, K, dev, seed)
    c = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    run = Launcher(tx, qa, qb, c, sa, sb, tx.SCALE_BLOCK128)
    iso, _ = time_cold(run, steps, warmup, flush)
    med = time_cold_in_stream(run, flush)
    warm = time_back_to_back(run, steps, warmup)
    nbytes = M * K + K * N + 2 * M * N + 4 * (sa.numel() + sb.numel())
    p = run.plan
    return dict(workload=f"fp8 e4m3 block-scaled decode M={M} N={N} K={K}", ms=med,
                ms_isolated=iso, ms_warm_mall=warm, gbps=nbytes / med / 1e6,
                frac_hbm=nbytes / med / 1e-3 / HBM, tflops=2.0 * M * N * K / med / 1e9,
                plan=plan_info(tx, p, split_k=p.split_k, grid=p.grid_x))


def bench_fp8(tx, dev, M, N, K, steps, warmup, seed=5, kmajor=False):
    """Config 4's block-scaled fp8 dot; kmajor: the weight kept [N][K] (B passed as its
    transpose), the layout a model's linear layer stores."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    a = torch.randn((M, K), generator=g, device=dev)
    b = torch.randn((K, N), generator=g, device=dev)
    kb, nb = (K + 127) // 128, (N + 127) // 128
    sa = a.view(M, kb, 128).abs().amax(dim=2) / 448.0
    sb = b.view(kb, 128, nb, 128).abs().amax(dim=(1, 3)) / 448.0
    qa = (a.view(M, kb, 128) / sa[:, :, None]).view(M, K).to(torch.float8_e4m3fn)
    qb = (b.view(kb, 128, nb, 128) / sb[:, None, :, None]).view(K, N).to(torch.float8_e4m3fn)
    if kmajor:
        qb = qb.t().contiguous().t()   # same values, K-major storage
    c = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    run = Launcher(tx, qa, qb, c, sa.contiguous(), sb.contiguous(), tx.SCALE_BLOCK128)
    assert bool(run.plan.desc.flags & tx.FLAG_B_KMAJOR) == kmajor
    ms = time_back_to_back(run, steps, warmup)
    flops = 2.0 * M * N * K
    return dict(workload=f"fp8 e4m3 block-scaled {M}x{N}x{K}" + (", B K-major" if kmajor else ""),
                ms=ms, tflops=flops / ms / 1e9,
                frac=flops / ms / 1e-3 / PEAK_I8, plan=plan_info(tx, run.plan))


def bench_vendor_decode(dev, flush, seed=1):
    """hipBLASLt on decode shapes at N = K = 8192, cold inside a stream like the decode
    lines, a reference point only: bf16 torch.matmul at M = 16 (bf16 C), and
    torch._int_mm (int32 C) at M = 32, the smallest M it takes above 16."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    N = K = 8192
    out = []
    a = torch.randn((16, K), generator=g, device=dev).to(torch.bfloat16)
    b = torch.randn((K, N), generator=g, device=dev).to(torch.bfloat16)
    c = torch.empty((16, N), dtype=torch.bfloat16, device=dev)
    ms = time_cold_in_stream(lambda: torch.matmul(a, b, out=c), flush)
    out.append(dict(workload=f"hipBLASLt (torch.matmul) bf16 M=16 N={N} K={K}", ms=ms,
                    gbps=(2 * 16 * K + 2 * K * N + 2 * 16 * N) / ms / 1e6))
    del b
    ai = torch.randint(-127, 128, (32, K), generator=g, device=dev, dtype=torch.int8)
    bi = torch.randint(-127, 128, (K, N), generator=g, device=dev, dtype=torch.int8)
    try:
        ms = time_cold_in_stream(lambda: torch._int_mm(ai, bi), flush)
        out.append(dict(workload=f"hipBLASLt (torch._int_mm) int8 M=32 N={N} K={K}, int32 C",
                        ms=ms, gbps=(32 * K + K * N + 4 * 32 * N) / ms / 1e6))
    except Exception as e:  # a torch build without the op: no vendor line, no failure
        print(f"# torch._int_mm: not available ({type(e).__name__})", file=sys.stderr)
    return out


def bench_fp8_unscaled(tx, dev, M, N, K, steps, warmup, seed=1):
    """fp8 e4m3 x e4m3 tt.dot with fp32 C (what the dot yields), B row-major: the
    256x256x128 tile, beside hipBLASLt's line of the same shape."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    a = torch.randn((M, K), generator=g, device=dev).to(torch.float8_e4m3fn)
    b = torch.randn((K, N), generator=g, device=dev).to(torch.float8_e4m3fn)
    c = torch.empty((M, N), dtype=torch.float32, device=dev)
    run = Launcher(tx, a, b, c)
    ms = time_back_to_back(run, steps, warmup)
    flops = 2.0 * M * N * K
    return dict(workload=f"fp8 e4m3 {M}x{N}x{K}, fp32 C", ms=ms, tflops=flops / ms / 1e9,
                frac=flops / ms / 1e-3 / PEAK_I8, plan=plan_info(tx, run.plan))


def mx_quantize(x, fmt):
    """OCP MX quantisation of x [R, K] along K: per 32 elements the shared
    exponent floor(log2(amax)) - emax (e4m3: 8, e2m1: 2), elements x / 2^e
    rounded to the format.  Returns (uint8 codes, e2m1 packed two per byte
    along K; uint8 e8m0 scales [R, K/32])."""
    import torch
    R, K = x.shape
    g = x.view(R, K // 32, 32)
    amax = g.abs().amax(dim=2).clamp_min(2.0 ** -100)
    e = torch.floor(torch.log2(amax)) - (8 if fmt == "e4m3" else 2)
    y = g / torch.exp2(e)[:, :, None]
    scales = (e + 127).clamp(0, 254).to(torch.uint8)
    if fmt == "e4m3":
        return y.reshape(R, K).to(torch.float8_e4m3fn).view(torch.uint8), scales
    vals = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], device=x.device)
    mid = (vals[1:] + vals[:-1]) / 2
    code = torch.bucketize(y.abs().clamp_max(6.0), mid).to(torch.uint8)
    code = (code | ((y < 0).to(torch.uint8) << 3)).reshape(R, K)
    return (code[:, 0::2] | (code[:, 1::2] << 4)).contiguous(), scales


def bench_mx(tx, dev, M, N, K, fmt, steps, warmup, seed=7):
    """tl.dot_scaled(A, sa, fmt, B, sb, fmt), fp32 C: N(0,1) inputs MX-quantised."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    qa, sa = mx_quantize(torch.randn((M, K), generator=g, device=dev), fmt)
    qbt, sb = mx_quantize(torch.randn((N, K), generator=g, device=dev), fmt)  # B^T rows
    # B [K, N] (e2m1: [K/2, N], byte (k2, n) = codes (2 k2, n) | (2 k2 + 1, n) << 4)
    qb = qbt.t().contiguous()
    c = torch.empty((M, N), dtype=torch.float32, device=dev)
    tf = tx.F8E4M3 if fmt == "e4m3" else tx.F4E2M1
    p = tx.plan(tx.make_desc(M, N, K, tf, tx.F32, scale_mode=tx.SCALE_MX32))
    L = tx.load()
    args = (ctypes.byref(p), qa.data_ptr(), qb.data_ptr(), c.data_ptr(), sa.data_ptr(),
            sb.data_ptr(), None, 0, torch.cuda.current_stream().cuda_stream)

    def run():
        rc = L.tx_dot_launch(*args)
        if rc != 0:
            raise RuntimeError(L.tx_get_last_error().decode())
    ms = time_back_to_back(run, steps, warmup)
    flops = 2.0 * M * N * K
    peak = PEAK_I8 if fmt == "e4m3" else PEAK_F4
    name = "mxfp8 e4m3" if fmt == "e4m3" else "mxfp4 e2m1"
    return dict(workload=f"tl.dot_scaled {name} (e8m0 per 32) {M}x{N}x{K}, fp32 C", ms=ms,
                tflops=flops / ms / 1e9, frac=flops / ms / 1e-3 / peak, peak_tflops=peak / 1e12,
                plan=plan_info(tx, p))


def bench_mx_bf16(tx, dev, M, N, K, fmt, steps, warmup, seed=8):
    """tl.dot_scaled(A bf16, None, "bf16", B, sb, fmt), fp32 C: B upcast to
    bf16 in the workspace, then the bf16 tile; both launches timed."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    a = torch.randn((M, K), generator=g, device=dev).to(torch.bfloat16)
    qbt, sb = mx_quantize(torch.randn((N, K), generator=g, device=dev), fmt)
    qb = qbt.t().contiguous()
    c = torch.empty((M, N), dtype=torch.float32, device=dev)
    tf = tx.F8E4M3 if fmt == "e4m3" else tx.F4E2M1
    p = tx.plan(tx.make_desc(M, N, K, tx.BF16, tx.F32, b_type=tf, scale_mode=tx.SCALE_MX32))
    ws = torch.empty(int(p.workspace_bytes), dtype=torch.uint8, device=dev)
    L = tx.load()
    args = (ctypes.byref(p), a.data_ptr(), qb.data_ptr(), c.data_ptr(), None, sb.data_ptr(),
            ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream)

    def run():
        rc = L.tx_dot_launch(*args)
        if rc != 0:
            raise RuntimeError(L.tx_get_last_error().decode())
    ms = time_back_to_back(run, steps, warmup)
    flops = 2.0 * M * N * K
    name = "mxfp8 e4m3" if fmt == "e4m3" else "mxfp4 e2m1"
    return dict(workload=f"tl.dot_scaled bf16 x {name} (upcast + bf16 tile) {M}x{N}x{K}, "
                         f"fp32 C", ms=ms, tflops=flops / ms / 1e9,
                frac=flops / ms / 1e-3 / PEAK_BF16, plan=plan_info(tx, p))


def bench_attn(tx, dev, N_CTX, causal, steps, warmup, Z=4, H=32, D=64, seed=9, dtype=None,
               block=(0, 0)):
    """Fused attention forward, the tutorial's bench_flash_attention "fwd"
    configuration (R:pass/LoopSplit/06-fused-attention.py:737-795): fp16
    randn q, k, v [4, 32, N_CTX, 64], sm_scale 1.3; FLOPs 4 Z H N^2 D, halved
    for causal.  block: (BLOCK_M, BLOCK_N), (0, 0) for the default."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    dtype = dtype or torch.float16
    fp8 = dtype == torch.float8_e5m2
    # the fp8 provider (:774-779): randn fp16 cast to e5m2, v stored key-contiguous
    q, k, v = (torch.randn((Z, H, N_CTX, D), generator=g, device=dev,
                           dtype=torch.float16 if fp8 else dtype).to(dtype) for _ in range(3))
    if fp8:
        v = v.permute(0, 1, 3, 2).contiguous().permute(0, 1, 3, 2)
    o = torch.empty_like(q, memory_format=torch.contiguous_format)
    M = torch.empty((Z, H, N_CTX), device=dev, dtype=torch.float32)
    p = tx.attn_plan(Z, H, N_CTX, D, causal, 1.3,
                     dtype=tx.F8E5M2 if fp8 else tx.BF16 if dtype == torch.bfloat16 else tx.F16,
                     strides={"v": (v.stride(0), v.stride(1), v.stride(3))} if fp8 else None,
                     block=block)
    L = tx.load()
    args = (ctypes.byref(p), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
            M.data_ptr(), torch.cuda.current_stream().cuda_stream)

    def run():
        rc = L.tx_attn_fwd_launch(*args)
        if rc != 0:
            raise RuntimeError(L.tx_get_last_error().decode())
    ms = time_back_to_back(run, steps, warmup)
    tn = "fp8 e5m2" if fp8 else "bf16" if dtype == torch.bfloat16 else "fp16"
    peak = PEAK_I8 if fp8 else PEAK_BF16  # fp8 MFMA peak = int8's 5.0 P
    blk = "" if block == (0, 0) else f" block={block[0]}x{block[1]}"
    return dict(workload=f"fused attention fwd {tn} Z={Z} H={H} N_CTX={N_CTX} D={D} "
                         f"causal={causal}{blk}", ms=ms, tflops=p.flops / ms / 1e9,
                frac=p.flops / ms / 1e-3 / peak)


def bench_vendor_attn(dev, N_CTX, causal, steps, warmup, Z=4, H=32, D=64, seed=9):
    # (fp16, as the tutorial's benchmark)
    """torch.nn.functional.scaled_dot_product_attention on the same inputs:
    the vendor reference (ROCm's fused attention behind torch)."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    q, k, v = (torch.randn((Z, H, N_CTX, D), generator=g, device=dev, dtype=torch.float16)
               for _ in range(3))
    fn = lambda: torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=causal,
                                                                  scale=1.3)
    ms = time_back_to_back(fn, steps, warmup)
    flops = 4.0 * Z * H * N_CTX * N_CTX * D * (0.5 if causal else 1.0)
    return dict(workload=f"vendor: torch sdpa fp16 Z={Z} H={H} N_CTX={N_CTX} D={D} "
                         f"causal={causal}", ms=ms, tflops=flops / ms / 1e9,
                frac=flops / ms / 1e-3 / PEAK_BF16)


def bench_int8(tx, dev, M, N, K, steps, warmup, seed=4):
    """int8 x int8 -> int32 tt.dot (no scales) on the 256x256x128 8-bit tile."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    a = torch.randint(-127, 128, (M, K), generator=g, device=dev, dtype=torch.int8)
    b = torch.randint(-127, 128, (K, N), generator=g, device=dev, dtype=torch.int8)
    c = torch.empty((M, N), dtype=torch.int32, device=dev)
    run = Launcher(tx, a, b, c)
    ms = time_back_to_back(run, steps, warmup)
    ops = 2.0 * M * N * K
    return dict(workload=f"int8 {M}x{N}x{K}, int32 C", ms=ms, tops=ops / ms / 1e9,
                frac=ops / ms / 1e-3 / PEAK_I8, plan=plan_info(tx, run.plan))


def ceilings_lib():
    """bench.py's hardware-ceiling kernels (triton-ext_amd/csrc/bench/ceilings.hip)."""
    L = ctypes.CDLL(os.path.join(ROOT, "triton-ext_amd", "lib", "libtx_ceilings.so"))
    vp = ctypes.c_void_p
    L.tx_ceiling_read.argtypes = [vp, ctypes.c_size_t, ctypes.c_int, vp, vp]
    L.tx_ceiling_mfma_bf16.argtypes = [vp, ctypes.c_int, ctypes.c_int, vp, vp]
    L.tx_ceiling_mfma_fp8.argtypes = [vp, ctypes.c_int, ctypes.c_int, vp, vp]
    L.tx_ceiling_mfma_bf16_stamped.argtypes = [vp, ctypes.c_int, ctypes.c_int, vp, vp, vp]
    L.tx_phases_bf16_setup.argtypes = [vp, ctypes.c_int]
    L.tx_phases_bf16.argtypes = [vp, vp, vp] + [ctypes.c_int] * 5 + [vp]
    L.tx_phases_8bit.argtypes = [ctypes.c_int, vp, vp, vp, vp, vp] + [ctypes.c_int] * 5 + [vp]
    L.tx_ceiling_mfma_fp8_stamped.argtypes = [vp, ctypes.c_int, ctypes.c_int, vp, vp, vp]
    L.tx_ceiling_operand_stream_8bit.argtypes = [vp, vp] + [ctypes.c_int] * 5 + [vp]
    return L


def bench_read_ceiling(dev, nbytes, steps, flush):
    """A plain streaming read of nbytes, timed like the W8A8 lines: cold inside a
    stream (after the 512 MiB read that evicts the MALL) and warm back to back.
    Variants: 16-byte loads 8 or 4 per thread (contiguous 32 / 16 KiB blocks), and
    direct-to-LDS loads through a per-wave ring as the decode kernel streams B."""
    import torch
    L = ceilings_lib()
    buf = torch.ones(nbytes // 4, dtype=torch.float32, device=dev)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    rows = []
    for variant, name in ((0, "16-byte loads x8, 32 KiB blocks"), (1, "16-byte loads x4, 16 KiB blocks"),
                          (2, "direct-to-LDS ring, 256 workgroups")):
        def run(v=variant):
            if L.tx_ceiling_read(buf.data_ptr(), nbytes, v, sink.data_ptr(), stream) != 0:
                raise RuntimeError("tx_ceiling_read failed")
        cold = time_cold_in_stream(run, flush)
        warm = time_back_to_back(run, steps, 3)
        rows.append(dict(variant=name, ms=cold, gbps=nbytes / cold / 1e6, ms_warm_mall=warm))
    best = min(rows, key=lambda r: r["ms"])
    return dict(workload=f"HBM read ceiling: plain read of {nbytes >> 20} MiB, cold, in stream",
                ms=best["ms"], gbps=best["gbps"], frac_hbm=best["gbps"] * 1e9 / HBM,
                variants=rows)


def bench_mfma_ceiling(dev, steps, warmup, seed=1, zeros=False):
    """The bf16 4096^3 tile schedule's MFMAs alone: 256 workgroups x 4 waves x 64 K
    steps x 64 v_mfma_f32_32x32x16_bf16, operands bf16 N(0,1)/64 (the headline's
    input distribution) held in registers.  zeros=True: all-zero operands, which toggle
    no operand bits -- the MFMA's power, and with it the clock, depends on them."""
    import torch
    L = ceilings_lib()
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    seed_t = (torch.randn((64 * 2048 * 8,), generator=g, device=dev) / 64).to(torch.bfloat16)
    if zeros:
        seed_t.zero_()
    out = torch.empty(256 * 256, dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream

    def run():
        if L.tx_ceiling_mfma_bf16(seed_t.data_ptr(), 256, 64, out.data_ptr(), stream) != 0:
            raise RuntimeError("tx_ceiling_mfma_bf16 failed")
    ms = time_back_to_back(run, steps, warmup)
    flops = 256 * 4 * 64 * 64 * 32768.0
    return dict(workload="MFMA ceiling: the bf16 4096^3 tile schedule's 2^22 "
                         "v_mfma_f32_32x32x16_bf16 alone (operands in registers"
                         + (", all zero)" if zeros else ", N(0,1)/64)"),
                ms=ms, tflops=flops / ms / 1e9, frac=flops / ms / 1e-3 / PEAK_BF16)


def phase_summary(w, ms, mfma_cyc):
    """Wave-time by phase from the stamps of a launch (16 words per wave: the wall clock at
    entry, step 0 landed, K loop done, epilogue issued, stores acknowledged, then XCC id,
    workgroup, and the shader clock at the same points), ms the launch period; mfma_cyc
    the MFMA cycles of one wave's K loop."""
    import numpy as np
    waves = w.shape[0]
    rt, sc = w[:, 0:5], w[:, 8:13]                 # wall clock (10 ns), shader clock
    r0, r4 = rt[:, 0].min(), rt[:, 4].max()
    T = ms * 1e3                                   # us per launch
    us = lambda x: x / 100.0
    loop_us = us(rt[:, 2] - rt[:, 1])
    loop_cyc = (sc[:, 2] - sc[:, 1]).astype(np.float64)
    mfma_us = loop_us * mfma_cyc / loop_cyc
    share = lambda x: round(float(np.sum(x)) / (waves * T), 4)
    mean = lambda x: round(float(np.mean(x)), 2)
    xcc = (w[:, 5] >> 32) & 7
    return dict(
        wave_time={
            "mfma_in_loop": share(mfma_us), "loop_other": share(loop_us - mfma_us),
            "before_entry": share(us(rt[:, 0] - r0)), "prologue": share(us(rt[:, 1] - rt[:, 0])),
            "epilogue": share(us(rt[:, 3] - rt[:, 2])),
            "store_drain": share(us(rt[:, 4] - rt[:, 3])),
            "after_own_end": share(us(r4 - rt[:, 4])),
            "between_launches": round(1.0 - us(r4 - r0) / T, 4)},
        us_mean={"prologue": mean(us(rt[:, 1] - rt[:, 0])), "k_loop": mean(loop_us),
                 "epilogue": mean(us(rt[:, 3] - rt[:, 2])),
                 "store_drain": mean(us(rt[:, 4] - rt[:, 3])),
                 "span": round(us(r4 - r0), 2), "launch": round(T, 2)},
        loop_ghz=round(float(np.mean(loop_cyc / (loop_us * 1e3))), 3),
        epilogue_ghz=round(float(np.mean((sc[:, 4] - sc[:, 2]) /
                                         (us(rt[:, 4] - rt[:, 2]) * 1e3))), 3),
        loop_mfma_busy=round(float(np.mean(mfma_cyc / loop_cyc)), 4),
        xcd_mean_end_us={int(x): mean(us(rt[xcc == x, 4] - r0)) for x in range(8)
                         if np.any(xcc == x)})


def bench_phases(dev, a, b, c, group_m, steps, warmup, seed=1):
    """Where one launch of the headline kernel goes.  libtx_ceilings.so builds
    gemm16_w4_kernel with its phase stamps on (per wave: the wall clock and the shader
    clock at entry, step 0 landed, K loop done, epilogue issued, stores acknowledged).
    The stamped kernel is timed back to back like the headline; the stamps of its last
    launch give each phase's share of the launch period in wave-time (one wave per SIMD
    here), the K loop's shader clock and its MFMA busy (2048 MFMA cycles per K step and
    wave against the loop's shader cycles).  A second pass stamps one K step at a time
    (its MFMA phase, its wait for loads and LDS reads, its barrier, in shader cycles),
    and the MFMA-only ceiling loop is stamped the same way for its clock and busy."""
    import numpy as np
    import torch
    L = ceilings_lib()
    M, K = a.shape
    N = b.shape[1]
    tm, tn, ks = M // 256, N // 256, K // 64
    waves = tm * tn * 4
    st = torch.zeros(waves * 16, dtype=torch.int64, device=dev)
    stream = torch.cuda.current_stream().cuda_stream

    def launch(n):
        if L.tx_phases_bf16(a.data_ptr(), b.data_ptr(), c.data_ptr(), tm, tn, ks, group_m, n,
                            stream) != 0:
            raise RuntimeError("tx_phases_bf16 failed")

    def stamps(probe):
        if L.tx_phases_bf16_setup(st.data_ptr(), probe) != 0:
            raise RuntimeError("tx_phases_bf16_setup failed")

    stamps(-1)
    ms = time_back_to_back(lambda: launch(1), steps, warmup)  # the last launch's stamps remain
    out = dict(workload="phases of the bf16 4096^3 tile, stamped build (libtx_ceilings.so)",
               ms_stamped=ms, tflops_stamped=2.0 * M * N * K / ms / 1e9)
    out.update(phase_summary(st.view(waves, 16).cpu().numpy().astype(np.int64), ms,
                             2048.0 * ks))
    mean = lambda x: round(float(np.mean(x)), 2)
    steps_probed = {}
    for s_ in (2, ks // 4, ks // 2, 3 * ks // 4, ks - 3):
        stamps(s_)
        launch(20)
        torch.cuda.synchronize()
        v = st.view(waves, 16).cpu().numpy().astype(np.int64)
        steps_probed[s_] = {"mfma_phase": mean(v[:, 13] - v[:, 7]),
                            "load_and_lds_wait": mean(v[:, 14] - v[:, 13]),
                            "barrier": mean(v[:, 15] - v[:, 14])}
    stamps(-1)
    out["step_cycles"] = steps_probed
    # the MFMA-only loop, stamped the same way
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    seed_t = (torch.randn((64 * 2048 * 8,), generator=g, device=dev) / 64).to(torch.bfloat16)
    cst = torch.zeros(1024 * 4, dtype=torch.int64, device=dev)
    cout = torch.empty(256 * 256, dtype=torch.float32, device=dev)

    def ceil():
        if L.tx_ceiling_mfma_bf16_stamped(seed_t.data_ptr(), 256, 64, cout.data_ptr(),
                                          cst.data_ptr(), stream) != 0:
            raise RuntimeError("tx_ceiling_mfma_bf16_stamped failed")
    cms = time_back_to_back(ceil, steps, warmup)
    cw = cst.view(1024, 4).cpu().numpy().astype(np.int64)
    c_us = (cw[:, 1] - cw[:, 0]) / 100.0
    c_cyc = (cw[:, 3] - cw[:, 2]).astype(np.float64)
    out["ceiling"] = {"ms": cms, "loop_ghz": round(float(np.mean(c_cyc / (c_us * 1e3))), 3),
                      "loop_mfma_busy": round(float(np.mean(2048.0 * 64 / c_cyc)), 4)}
    return out


def bench_phases8(dev, steps, warmup, seed=5):
    """Where a launch of the 8-bit 256x256x128 tile goes, for C5 (fp8 block-scaled
    2048x7168x7168, bf16 C), int8 4096^3 (int32 C) and MX e4m3 / e2m1 4096^3 (fp32 C):
    libtx_ceilings.so builds gemm8_w4_kernel with its phase stamps on, as bench_phases
    does for the bf16 tile.  A wave runs 8 x 4 blocks a step (128 bytes of K), one
    v_mfma_f32_16x16x128_f8f6f4 (fp8), two v_mfma_i32_16x16x64_i8 (int8) or two
    e2m1 v_mfma_scale_f32_16x16x128_f8f6f4 each: 1024 MFMA cycles a step, two waves a
    SIMD.  The C5 schedule's MFMA-only ceiling loop is stamped alike for its clock and
    busy."""
    import numpy as np
    import torch
    L = ceilings_lib()
    stream = torch.cuda.current_stream().cuda_stream
    out = []
    for kind, (M, N, K) in ((0, (2048, 7168, 7168)), (1, (4096, 4096, 4096)),
                            (2, (4096, 4096, 4096)), (3, (4096, 4096, 4096))):
        kb = K // 2 if kind == 3 else K  # bytes of K (e2m1: two per byte)
        if kind >= 2:
            fmt = "e4m3" if kind == 2 else "e2m1"
            g = torch.Generator(device=dev)
            g.manual_seed(seed)
            a, sa = mx_quantize(torch.randn((M, K), generator=g, device=dev), fmt)
            qbt, sb = mx_quantize(torch.randn((N, K), generator=g, device=dev), fmt)
            b = qbt.t().contiguous()
            c = torch.empty((M, N), dtype=torch.float32, device=dev)
            name = f"MX {fmt} (e8m0 per 32, fp32 C)"
        elif kind == 0:
            a, b, sa, sb = fp8_block_inputs_dev(M, N, K, dev, seed)
            c = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
            name = "fp8 block-scaled (C5)"
        else:
            g = torch.Generator(device=dev)
            g.manual_seed(seed)
            a = torch.randint(-127, 128, (M, K), generator=g, device=dev, dtype=torch.int8)
            b = torch.randint(-127, 128, (K, N), generator=g, device=dev, dtype=torch.int8)
            sa = sb = None
            c = torch.empty((M, N), dtype=torch.int32, device=dev)
            name = "int8 -> int32"
        tm, tn, ks = M // 256, N // 256, kb // 128
        waves = tm * tn * 8
        st = torch.zeros(waves * 16, dtype=torch.int64, device=dev)
        if L.tx_phases_bf16_setup(st.data_ptr(), -1) != 0:
            raise RuntimeError("tx_phases_bf16_setup failed")

        def launch():
            if L.tx_phases_8bit(kind, a.data_ptr(), b.data_ptr(), c.data_ptr(),
                                None if sa is None else sa.data_ptr(),
                                None if sb is None else sb.data_ptr(), tm, tn, ks, 4, 1,
                                stream) != 0:
                raise RuntimeError("tx_phases_8bit failed")
        ms = time_back_to_back(launch, steps, warmup)
        r = dict(workload=f"phases of the 8-bit 256x256x128 tile, {name} {M}x{N}x{K}, stamped build",
                 ms_stamped=ms, tflops_stamped=2.0 * M * N * K / ms / 1e9)
        w = st.view(waves, 16).cpu().numpy().astype(np.int64)
        r.update(phase_summary(w, ms, 1024.0 * ks))
        del r["loop_mfma_busy"]  # a wave's share means little with two waves on a SIMD
        # The two waves of a SIMD (same XCC, SE, SH, CU and SIMD id in HW_ID): both waves'
        # MFMA cycles over the union of their K loops, on the CU's shader clock.
        h = w[:, 5]
        key = (((h >> 32) & 7) << 16) | (((h >> 13) & 7) << 12) | (((h >> 12) & 1) << 11) | \
              (((h >> 8) & 15) << 4) | ((h >> 4) & 3)
        busy = []
        for k in np.unique(key):
            sel = w[key == k]
            span = float(sel[:, 10].max() - sel[:, 9].min())
            busy.append(1024.0 * ks * len(sel) / span)
        r["simd_mfma_busy_in_loop"] = round(float(np.mean(busy)), 4)
        r["waves_per_simd"] = round(waves / len(busy), 2)
        # single K steps: the MFMA phase (a step's 32 blocks), the wait for the next
        # step's loads and the LDS reads, the barrier; shader cycles, mean over waves
        mean = lambda x: round(float(np.mean(x)), 2)
        probed = {}
        for s_ in (2, ks // 2, ks - 3):
            if L.tx_phases_bf16_setup(st.data_ptr(), s_) != 0:
                raise RuntimeError("tx_phases_bf16_setup failed")
            for _ in range(20):
                launch()
            torch.cuda.synchronize()
            v = st.view(waves, 16).cpu().numpy().astype(np.int64)
            probed[s_] = {"mfma_phase": mean(v[:, 13] - v[:, 7]),
                          "load_and_lds_wait": mean(v[:, 14] - v[:, 13]),
                          "barrier": mean(v[:, 15] - v[:, 14])}
        if L.tx_phases_bf16_setup(st.data_ptr(), -1) != 0:
            raise RuntimeError("tx_phases_bf16_setup failed")
        r["step_cycles"] = probed

        # the tile's A and B loads alone (its load code, order and step barrier)
        def stream_only():
            if L.tx_ceiling_operand_stream_8bit(a.data_ptr(), b.data_ptr(), tm, tn, ks, 4, 1,
                                                stream) != 0:
                raise RuntimeError("tx_ceiling_operand_stream_8bit failed")
        sms = time_back_to_back(stream_only, steps, warmup)
        r["operand_stream"] = {"ms": sms, "gb_per_s_per_cu": round(ks * 65536 / sms / 1e6, 1)}
        out.append(r)
    g = torch.Generator(device=dev)
    g.manual_seed(2)
    vals = (torch.randn((64 * 12 * 64 * 32,), generator=g, device=dev) * 100).clamp(-448, 448)
    seed_t = vals.to(torch.float8_e4m3fn).view(torch.uint8)
    cout = torch.empty(224 * 512, dtype=torch.float32, device=dev)
    cst = torch.zeros(224 * 8 * 4, dtype=torch.int64, device=dev)

    def ceil():
        if L.tx_ceiling_mfma_fp8_stamped(seed_t.data_ptr(), 224, 56, cout.data_ptr(),
                                         cst.data_ptr(), stream) != 0:
            raise RuntimeError("tx_ceiling_mfma_fp8_stamped failed")
    cms = time_back_to_back(ceil, steps, warmup)
    cw = cst.view(224, 8, 4).cpu().numpy().astype(np.int64)
    c_us = (cw[:, :, 1] - cw[:, :, 0]) / 100.0
    c_cyc = (cw[:, :, 3] - cw[:, :, 2]).astype(np.float64)
    # waves w and w + 4 of a workgroup share SIMD w: the union of their loops
    span = np.maximum(cw[:, :4, 3], cw[:, 4:, 3]) - np.minimum(cw[:, :4, 2], cw[:, 4:, 2])
    out[0]["ceiling"] = {"ms": cms, "loop_ghz": round(float(np.mean(c_cyc / (c_us * 1e3))), 3),
                         "simd_mfma_busy_in_loop": round(float(np.mean(2 * 1024.0 * 56 / span)), 4)}
    return out


def bench_mfma_ceiling_fp8(dev, steps, warmup, seed=2, zeros=False):
    """The fp8 C5 tile schedule's MFMAs alone: 224 workgroups (C5's 8 x 28 tiles) x 8
    waves x 56 K steps x 32 v_mfma_f32_16x16x128_f8f6f4, e4m3 operands held in registers:
    codes of N(0,1) * 100 (saturated at 448, no NaN codes), spread over the e4m3 range
    as C5's amax/448-quantised values are; zeros=True: all-zero operands."""
    import torch
    L = ceilings_lib()
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    vals = (torch.randn((64 * 12 * 64 * 32,), generator=g, device=dev) * 100).clamp(-448, 448)
    seed_t = vals.to(torch.float8_e4m3fn).view(torch.uint8)
    if zeros:
        seed_t.zero_()
    out = torch.empty(224 * 512, dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream

    def run():
        if L.tx_ceiling_mfma_fp8(seed_t.data_ptr(), 224, 56, out.data_ptr(), stream) != 0:
            raise RuntimeError("tx_ceiling_mfma_fp8 failed")
    ms = time_back_to_back(run, steps, warmup)
    flops = 224 * 8 * 56 * 32 * 65536.0
    return dict(workload="fp8 MFMA ceiling: the C5 tile schedule's v_mfma_f32_16x16x128_f8f6f4 "
                         "alone (224 workgroups, operands in registers"
                         + (", all zero)" if zeros else ", e4m3 of N(0,1)*100)"),
                ms=ms, tflops=flops / ms / 1e9, frac=flops / ms / 1e-3 / PEAK_I8)


def bench_tiles(tx, dev, steps, warmup):
    """Every instantiated tile at one large shape per operand type: the measured
    sustained fraction of peak behind the arith_intensity pass's tile weights."""
    import torch
    rows = []
    M = N = K = 4096
    a, b = bf16_inputs(M, N, K, dev, 11)
    c = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    for blk in ((256, 256, 64), (128, 128, 64), (64, 64, 32)):
        run = Launcher(tx, a, b, c, block=blk)
        ms = time_back_to_back(run, steps, warmup)
        rows.append(dict(workload=f"tile {blk[0]}x{blk[1]}x{blk[2]} bf16 4096^3", tile=list(blk),
                         ms=ms, tflops=2.0 * M * N * K / ms / 1e9,
                         frac=2.0 * M * N * K / ms / 1e-3 / PEAK_BF16, plan=plan_info(tx, run.plan)))
    g = torch.Generator(device=dev)
    g.manual_seed(12)
    ai = torch.randint(-127, 128, (M, K), generator=g, device=dev, dtype=torch.int8)
    bi = torch.randint(-127, 128, (K, N), generator=g, device=dev, dtype=torch.int8)
    ci = torch.empty((M, N), dtype=torch.int32, device=dev)
    for blk in ((256, 256, 128), (256, 224, 128), (128, 128, 128)):
        run = Launcher(tx, ai, bi, ci, block=blk)
        ms = time_back_to_back(run, steps, warmup)
        rows.append(dict(workload=f"tile {blk[0]}x{blk[1]}x{blk[2]} int8 4096^3", tile=list(blk),
                         ms=ms, tops=2.0 * M * N * K / ms / 1e9,
                         frac=2.0 * M * N * K / ms / 1e-3 / PEAK_I8, plan=plan_info(tx, run.plan)))
    return rows


def cpu_baseline(a, b, c, M, N, K, block):
    """Oracle on the host cores over the full bf16 workload; also checks the GPU output."""
    import numpy as np
    import torch

    import oracle
    ha = a.view(torch.int16).cpu().numpy().view(np.uint16)
    hb = b.view(torch.int16).cpu().numpy().view(np.uint16)
    got = c.view(torch.int16).cpu().numpy().view(np.uint16)
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    t0 = time.perf_counter()
    ref = oracle.tiled_dot(ha, hb, a_type=oracle.BF16, c_type=oracle.BF16, block=block,
                           nthreads=threads)
    dt = time.perf_counter() - t0
    g32, r32 = oracle.bf16_to_f32(got).astype(np.float64), oracle.bf16_to_f32(ref).astype(np.float64)
    ok = bool((np.abs(g32 - r32) <= 1e-3 + 1e-2 * np.abs(r32)).all())
    cpu = open("/proc/cpuinfo").read() if os.path.exists("/proc/cpuinfo") else ""
    model = next((ln.split(":", 1)[1].strip() for ln in cpu.splitlines() if ln.startswith("model name")), "?")
    return dict(value=2.0 * M * N * K / dt / 1e12, unit="TFLOP/s", cores=threads, kind="port",
                sample=f"full bf16 {M}x{N}x{K} dot, {block[0]}x{block[1]}x{block[2]} tiles, "
                       f"{dt:.2f} s on {threads} threads ({model})",
                seconds=dt), ok


def copy_probe():
    import torch
    x = torch.ones((256 << 20) // 4, dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    for _ in range(5):
        y.copy_(x)
    torch.cuda.synchronize()
    print("copied 5 x 256 MiB", flush=True)


def main():
    args = parse()
    if args.copy_probe:
        copy_probe()
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(a dot would shard by blocks of N or M columns/rows, one per GPU, with no "
              "exchange between them).", file=sys.stderr)
        sys.exit(2)
    import torch

    import triton_ext_amd as tx
    dev = torch.device("cuda:0")
    if not tx.load().tx_device_available():
        print("cuda:0 is not a gfx950 device", file=sys.stderr)
        sys.exit(3)
    only = set(x for x in args.only.split(",") if x)

    def want(name):
        return not only or name in only

    M = N = K = 4096
    head, (a, b, c) = bench_bf16(tx, dev, M, N, K, args.steps, args.warmup)
    print(f"# bf16 4096^3: {head['ms'] * 1e3:.1f} us/step, {head['tflops']:.1f} TFLOP/s, "
          f"{100 * head['frac']:.1f}% of peak", file=sys.stderr, flush=True)
    secondary = []
    if want("vendor"):
        r = bench_vendor_bf16(dev, M, N, K, args.steps, args.warmup)
        secondary.append(r)
        print(f"# {r['workload']}: {r['tflops']:.1f} TFLOP/s", file=sys.stderr, flush=True)
    if want("vendor") or want("vendor8"):
        for r in bench_vendor_8bit(dev, args.steps, args.warmup):
            secondary.append(r)
            print(f"# {r['workload']}: {r['tflops']:.1f} T/s", file=sys.stderr, flush=True)
    if want("c1"):
        r = bench_c1(tx, dev, args.steps, args.warmup)
        secondary.append(r)
        print(f"# {r['workload']}: {r['ms'] * 1e3:.2f} us, {r['tflops']:.1f} TFLOP/s",
              file=sys.stderr, flush=True)
    if want("kmajor"):
        r = bench_bf16_kmajor(tx, dev, M, N, K, args.steps, args.warmup)
        secondary.append(r)
        print(f"# {r['workload']}: {r['tflops']:.1f} TFLOP/s", file=sys.stderr, flush=True)
        for kind in ("int8", "fp8"):
            r = bench_8bit_kmajor(tx, dev, kind, 4096, 4096, 4096, args.steps, args.warmup)
            secondary.append(r)
            print(f"# {r['workload']}: {r['ms'] * 1e3:.1f} us, {r['tops']:.1f} T/s",
                  file=sys.stderr, flush=True)
        r = bench_fp8(tx, dev, 2048, 7168, 7168, args.steps, args.warmup, kmajor=True)
        secondary.append(r)
        print(f"# {r['workload']}: {r['ms'] * 1e3:.1f} us, {r['tflops']:.1f} TFLOP/s",
              file=sys.stderr, flush=True)
    flush = make_flush(dev)
    if want("tail"):
        for (m, n, k) in ((4096, 4096, 4000), (4000, 4000, 4000)):
            r, _ = bench_bf16(tx, dev, m, n, k, args.steps, args.warmup, seed=2)
            secondary.append(r)
            print(f"# {r['workload']}: {r['tflops']:.1f} TFLOP/s", file=sys.stderr, flush=True)
    if want("tiles"):
        for r in bench_tiles(tx, dev, args.steps, args.warmup):
            secondary.append(r)
            print(f"# {r['workload']}: {100 * r['frac']:.1f}% of peak", file=sys.stderr, flush=True)
    if want("phases"):
        r = bench_phases(dev, a, b, c, head["plan"]["group_m"], args.steps, args.warmup)
        secondary.append(r)
        f = r["wave_time"]
        print(f"# {r['workload']}: {r['ms_stamped'] * 1e3:.1f} us/launch; wave-time: MFMA in loop "
              f"{100 * f['mfma_in_loop']:.1f}%, loop other {100 * f['loop_other']:.1f}%, prologue "
              f"{100 * f['prologue']:.1f}%, epilogue {100 * f['epilogue']:.1f}% + drain "
              f"{100 * f['store_drain']:.1f}%, skew {100 * (f['before_entry'] + f['after_own_end']):.1f}%, "
              f"between launches {100 * f['between_launches']:.1f}%; loop {r['loop_ghz']:.2f} GHz, "
              f"{100 * r['loop_mfma_busy']:.1f}% MFMA busy (ceiling loop {r['ceiling']['loop_ghz']:.2f} GHz, "
              f"{100 * r['ceiling']['loop_mfma_busy']:.1f}%); per step (cycles) "
              + ", ".join(f"{k}: {v['mfma_phase']:.0f}+{v['load_and_lds_wait']:.0f}+{v['barrier']:.0f}"
                          for k, v in r["step_cycles"].items()),
              file=sys.stderr, flush=True)
    if "phases8" in only:
        for r in bench_phases8(dev, args.steps, args.warmup):
            secondary.append(r)
            f = r["wave_time"]
            print(f"# {r['workload']}: {r['ms_stamped'] * 1e3:.1f} us/launch "
                  f"({r['tflops_stamped']:.0f} T/s); wave-time: MFMA in loop "
                  f"{100 * f['mfma_in_loop']:.1f}%, loop other {100 * f['loop_other']:.1f}%, "
                  f"prologue {100 * f['prologue']:.1f}%, epilogue {100 * f['epilogue']:.1f}% + "
                  f"drain {100 * f['store_drain']:.1f}%, skew "
                  f"{100 * (f['before_entry'] + f['after_own_end']):.1f}%, between launches "
                  f"{100 * f['between_launches']:.1f}%; loop {r['loop_ghz']:.2f} GHz, SIMD "
                  f"{100 * r['simd_mfma_busy_in_loop']:.1f}% MFMA busy"
                  + (f" (ceiling loop {r['ceiling']['loop_ghz']:.2f} GHz, "
                     f"{100 * r['ceiling']['simd_mfma_busy_in_loop']:.1f}%)" if "ceiling" in r else "")
                  + "; per step (cycles) "
                  + ", ".join(f"{k}: {v['mfma_phase']:.0f}+{v['load_and_lds_wait']:.0f}+{v['barrier']:.0f}"
                              for k, v in r["step_cycles"].items())
                  + f"; A and B loads alone {r['operand_stream']['ms'] * 1e3:.1f} us "
                  f"({r['operand_stream']['gb_per_s_per_cu']:.1f} GB/s per CU)",
                  file=sys.stderr, flush=True)
    ceil = {}
    if want("ceiling"):
        for zeros in (False, True):
            r = bench_mfma_ceiling(dev, args.steps, args.warmup, zeros=zeros)
            secondary.append(r)
            ceil["mfma_bf16_zero_operands_tflops" if zeros else "mfma_bf16_tflops"] = \
                round(r["tflops"], 1)
            print(f"# {r['workload']}: {r['tflops']:.1f} TFLOP/s ({100 * r['frac']:.1f}% of spec)",
                  file=sys.stderr, flush=True)
        for zeros in (False, True):
            r = bench_mfma_ceiling_fp8(dev, args.steps, args.warmup, zeros=zeros)
            secondary.append(r)
            ceil["mfma_fp8_zero_operands_tflops" if zeros else "mfma_fp8_tflops"] = \
                round(r["tflops"], 1)
            print(f"# {r['workload']}: {r['tflops']:.1f} TFLOP/s ({100 * r['frac']:.1f}% of spec)",
                  file=sys.stderr, flush=True)
        for nb in (64 << 20, 1 << 30):
            r = bench_read_ceiling(dev, nb, max(args.steps, 20), flush)
            secondary.append(r)
            ceil[f"hbm_read_{nb >> 20}MiB_gbps"] = round(r["gbps"], 1)
            print(f"# {r['workload']}: {r['ms'] * 1e3:.2f} us, {r['gbps']:.0f} GB/s "
                  f"({100 * r['frac_hbm']:.1f}% of 8 TB/s); "
                  + ", ".join(f"{v['variant']}: {v['gbps']:.0f}" for v in r["variants"]),
                  file=sys.stderr, flush=True)
    w8a8_ms = [m for m in (1, 16, 64, 256) if want("w8a8") or want(f"w8a8_{m}")]
    w8a8_16 = None
    if w8a8_ms:
        for m in w8a8_ms:
            r = bench_w8a8(tx, dev, m, 8192, 8192, max(args.steps, 20), 3, flush)
            secondary.append(r)
            if m == 16:
                w8a8_16 = r
            print(f"# {r['workload']}: {r['ms'] * 1e3:.2f} us in stream, {r['gbps']:.0f} GB/s "
                  f"({100 * r['frac_hbm']:.1f}% HBM); isolated launch "
                  f"{r['ms_isolated'] * 1e3:.2f} us", file=sys.stderr, flush=True)
    for m in (1, 16, 64, 256):
        if want("w8a8_kmajor") or want(f"w8a8_kmajor_{m}"):
            r = bench_w8a8(tx, dev, m, 8192, 8192, max(args.steps, 20), 3, flush, kmajor=True)
            secondary.append(r)
            print(f"# {r['workload']}: {r['ms'] * 1e3:.2f} us in stream, {r['gbps']:.0f} GB/s "
                  f"({100 * r['frac_hbm']:.1f}% HBM); isolated launch "
                  f"{r['ms_isolated'] * 1e3:.2f} us", file=sys.stderr, flush=True)
    for km in (False, True):
        if want("w8a8") or want("i32_16_kmajor" if km else "i32_16"):
            r = bench_decode_i32(tx, dev, 16, 8192, 8192, max(args.steps, 20), 3, flush, kmajor=km)
            secondary.append(r)
            print(f"# {r['workload']}: {r['ms'] * 1e3:.2f} us in stream, {r['gbps']:.0f} GB/s "
                  f"({100 * r['frac_hbm']:.1f}% HBM)", file=sys.stderr, flush=True)
    for m in (1, 16, 64):
        if want("fp8_decode") or want(f"fp8_decode_{m}"):
            r = bench_decode_f8(tx, dev, m, 7168, 7168, max(args.steps, 20), 3, flush)
            secondary.append(r)
            print(f"# {r['workload']}: {r['ms'] * 1e3:.2f} us in stream, {r['gbps']:.0f} GB/s "
                  f"({100 * r['frac_hbm']:.1f}% HBM); isolated launch "
                  f"{r['ms_isolated'] * 1e3:.2f} us", file=sys.stderr, flush=True)
    if want("vendor") or want("vendor_decode"):
        for r in bench_vendor_decode(dev, flush):
            secondary.append(r)
            print(f"# {r['workload']}: {r['ms'] * 1e3:.2f} us in stream, {r['gbps']:.0f} GB/s",
                  file=sys.stderr, flush=True)
    for m, km in ((1, False), (16, False), (64, False), (96, False), (1, True), (16, True),
                  (64, True), (96, True)):
        name = "bf16_decode_kmajor" if km else "bf16_decode"
        if want(name) or want(f"{name}_{m}"):
            r = bench_decode16(tx, dev, m, 8192, 8192, max(args.steps, 20), 3, flush, kmajor=km)
            secondary.append(r)
            print(f"# {r['workload']}: {r['ms'] * 1e3:.2f} us in stream, {r['gbps']:.0f} GB/s "
                  f"({100 * r['frac_hbm']:.1f}% HBM); isolated launch "
                  f"{r['ms_isolated'] * 1e3:.2f} us", file=sys.stderr, flush=True)
    if only and "decode16_widths" in only:
        for r in bench_decode16_widths(tx, dev, flush):
            secondary.append(r)
            print(f"# {r['workload']}: {r['ms_w64'] * 1e3:.1f} / {r['ms_w128'] * 1e3:.1f} us in "
                  f"stream", file=sys.stderr, flush=True)
    for kind, m, n in (("bf16", 128, 8192), ("bf16", 256, 8192), ("bf16", 512, 8192),
                       ("fp8", 256, 7168)):
        if want("mid_m") or want(f"mid_m_{kind}_{m}"):
            r = bench_mid_m(tx, dev, kind, m, n, n, flush)
            secondary.append(r)
            v = f"; hipBLASLt {r['ms_vendor'] * 1e3:.1f} us" if r["ms_vendor"] else ""
            print(f"# {r['workload']} (split {r['plan']['split_k']}): {r['ms'] * 1e3:.1f} us in "
                  f"stream, {r['tflops']:.0f} TFLOP/s{v}", file=sys.stderr, flush=True)
    if want("int8"):
        r = bench_int8(tx, dev, 4096, 4096, 4096, args.steps, args.warmup)
        secondary.append(r)
        print(f"# {r['workload']}: {r['tops']:.1f} TOP/s ({100 * r['frac']:.1f}% of 5033)",
              file=sys.stderr, flush=True)
    if want("fp8"):
        r = bench_fp8(tx, dev, 2048, 7168, 7168, args.steps, args.warmup)
        secondary.append(r)
        print(f"# {r['workload']}: {r['tflops']:.1f} TFLOP/s", file=sys.stderr, flush=True)
    if want("fp8") or want("fp8u"):
        r = bench_fp8_unscaled(tx, dev, 4096, 4096, 4096, args.steps, args.warmup)
        secondary.append(r)
        print(f"# {r['workload']}: {r['tflops']:.1f} TFLOP/s ({100 * r['frac']:.1f}% of 5033)",
              file=sys.stderr, flush=True)

    for fmt, short in (("e4m3", "mxfp8"), ("e2m1", "mxfp4")):
        for n in (4096, 8192):
            if want("mx") or want(short) or want(f"{short}_{n}"):
                r = bench_mx(tx, dev, n, n, n, fmt, args.steps, args.warmup)
                secondary.append(r)
                print(f"# {r['workload']}: {r['tflops']:.1f} TFLOP/s "
                      f"({100 * r['frac']:.1f}% of {r['peak_tflops']:.0f})", file=sys.stderr,
                      flush=True)

    for fmt, short in (("e2m1", "mxbf16_fp4"), ("e4m3", "mxbf16_fp8")):
        if want("mxbf16") or want(short):
            r = bench_mx_bf16(tx, dev, 4096, 4096, 4096, fmt, args.steps, args.warmup)
            secondary.append(r)
            print(f"# {r['workload']}: {r['tflops']:.1f} TFLOP/s "
                  f"({100 * r['frac']:.1f}% of bf16 peak)", file=sys.stderr, flush=True)

    for n in (1024, 4096, 16384):
        if want("attn") or want(f"attn_{n}"):
            for causal in (True, False):
                r = bench_attn(tx, dev, n, causal, args.steps, args.warmup)
                secondary.append(r)
                print(f"# {r['workload']}: {r['tflops']:.1f} TFLOP/s "
                      f"({100 * r['frac']:.1f}% of fp16 peak)", file=sys.stderr, flush=True)
                if want("vendor") or want("attn_vendor"):
                    r = bench_vendor_attn(dev, n, causal, args.steps, args.warmup)
                    secondary.append(r)
                    print(f"# {r['workload']}: {r['tflops']:.1f} TFLOP/s", file=sys.stderr,
                          flush=True)

    for n in (1024, 4096, 16384):  # the tutorial's "triton-fp8" provider
        if want("attn_fp8") or want(f"attn_fp8_{n}"):
            for causal in (True, False):
                r = bench_attn(tx, dev, n, causal, args.steps, args.warmup,
                               dtype=torch.float8_e5m2)
                secondary.append(r)
                print(f"# {r['workload']}: {r['tflops']:.1f} TFLOP/s "
                      f"({100 * r['frac']:.1f}% of fp8 peak)", file=sys.stderr, flush=True)

    if want("attn_d128"):  # head dim 128 (beyond the tutorial's 64), fp16 and e5m2
        for causal in (True, False):
            r = bench_attn(tx, dev, 4096, causal, args.steps, args.warmup, Z=4, H=16, D=128)
            secondary.append(r)
            print(f"# {r['workload']}: {r['tflops']:.1f} TFLOP/s", file=sys.stderr, flush=True)
            r = bench_attn(tx, dev, 4096, causal, args.steps, args.warmup, Z=4, H=16, D=128,
                           dtype=torch.float8_e5m2)
            secondary.append(r)
            print(f"# {r['workload']}: {r['tflops']:.1f} TFLOP/s", file=sys.stderr, flush=True)
            if want("vendor") or want("attn_vendor"):
                r = bench_vendor_attn(dev, 4096, causal, args.steps, args.warmup, Z=4, H=16, D=128)
                secondary.append(r)
                print(f"# {r['workload']}: {r['tflops']:.1f} TFLOP/s", file=sys.stderr,
                      flush=True)

    cpu, parity = None, None
    if not args.no_cpu:
        # recompute the headline output once more (the secondary runs reused no buffers)
        Launcher(tx, a, b, c)()
        torch.cuda.synchronize()
        tile = head["plan"]["tile"]
        cpu, parity = cpu_baseline(a, b, c, M, N, K, tuple(tile))
        print(f"# cpu baseline: {cpu['value']:.3f} TFLOP/s, parity={parity}", file=sys.stderr, flush=True)

    flops = 2.0 * M * N * K
    line = {
        "metric": METRIC, "value": round(head["tflops"], 2), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(head["ms"], 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (torch.randn / sqrt(K), seed 1, rounded to bf16)",
        "config": {"workload": "bf16 dense dot C=A@B, M=N=K=4096, row-major A[M,K], B[K,N], "
                               "fp32 accumulate, bf16 out (BASELINE configs[1])",
                   "tile": head["plan"]["tile"], "kernel": "gemm16_w4_kernel<bf16, 4 waves of 128x128>",
                   "intensity": head["plan"]["intensity"], "classified": head["plan"]["bound"]},
        "roofline": {"bound": "mfma", "achieved": round(flops / head["ms"] / 1e9, 2),
                     "peak": PEAK_BF16 / 1e12, "unit": "TFLOP/s", "frac": round(head["frac"], 4),
                     "traffic": TRAFFIC_BF16_4096},
        "cpu_baseline": cpu if cpu is None else {k: v for k, v in cpu.items() if k != "seconds"},
        # the metric's second half: W8A8 decode at M=16 (N=K=8192), a cold launch inside a
        # stream, algorithmic bytes (B, A, scales and C once) over its time
        "roofline_w8a8_m16": None if w8a8_16 is None else {
            "bound": "hbm", "achieved": round(w8a8_16["gbps"], 1), "peak": HBM / 1e9,
            "unit": "GB/s", "frac": round(w8a8_16["frac_hbm"], 4), "traffic": TRAFFIC_W8A8_M16,
            "ms": round(w8a8_16["ms"], 5)},
        "ceilings": ceil or None,
        "parity_vs_oracle": parity,
        "secondary": secondary,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
