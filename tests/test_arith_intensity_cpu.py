"""arith_intensity classifier vs closed forms (BASELINE figures)."""
import pytest

import triton_ext_amd as tx

PEAK16, PEAK8, HBM = 2516.6e12, 5033.2e12, 8.0e12


@pytest.mark.parametrize("M,N,K,a,c,sm,flops,nbytes,bound", [
    (4096, 4096, 4096, tx.BF16, tx.BF16, 0, 2 * 4096**3, 3 * 4096 * 4096 * 2, tx.BOUND_MFMA),
    (4096, 4096, 4000, tx.BF16, tx.BF16, 0, 2 * 4096 * 4096 * 4000,
     4096 * 4000 * 2 * 2 + 4096 * 4096 * 2, tx.BOUND_MFMA),
    (512, 512, 512, tx.F16, tx.F32, 0, 2 * 512**3, 512 * 512 * (2 + 2 + 4), tx.BOUND_HBM),
    (16, 8192, 8192, tx.I8, tx.BF16, tx.SCALE_ROWCOL, 2 * 16 * 8192 * 8192,
     16 * 8192 + 8192 * 8192 + 16 * 8192 * 2 + 4 * (16 + 8192), tx.BOUND_HBM),
    (256, 8192, 8192, tx.I8, tx.BF16, tx.SCALE_ROWCOL, 2 * 256 * 8192 * 8192,
     256 * 8192 + 8192 * 8192 + 256 * 8192 * 2 + 4 * (256 + 8192), tx.BOUND_HBM),
    (2048, 7168, 7168, tx.F8E4M3, tx.BF16, tx.SCALE_BLOCK128, 2 * 2048 * 7168 * 7168,
     2048 * 7168 + 7168 * 7168 + 2048 * 7168 * 2 + 4 * (2048 * 56 + 56 * 56), tx.BOUND_MFMA),
])
def test_closed_form(M, N, K, a, c, sm, flops, nbytes, bound):
    r = tx.arith_intensity(tx.make_desc(M, N, K, a, c, scale_mode=sm))
    assert r.flops == flops
    assert r.bytes == nbytes
    assert r.intensity == pytest.approx(flops / nbytes)
    peak = PEAK16 if a in (tx.BF16, tx.F16) else PEAK8
    assert r.peak_flops == peak and r.peak_bw == HBM
    assert r.ridge == pytest.approx(peak / HBM)
    assert r.bound == bound
    assert r.roofline_us == pytest.approx(1e6 * max(flops / peak, nbytes / HBM))
    es = 2 if a in (tx.BF16, tx.F16) else 1
    assert r.tile_intensity == pytest.approx(
        2 * r.block_m * r.block_n / ((r.block_m + r.block_n) * es))


def test_baseline_roofline_times():
    """Roofline times of the benchmark configs at the MI355X peaks (bf16 4096^3 at
    2516.6 TFLOP/s, W8A8 M=16 and fp8 C5 at 8 TB/s and 5033 TFLOP/s respectively)."""
    cases = [((4096, 4096, 4096, tx.BF16, tx.BF16, 0), 54.6),
             ((16, 8192, 8192, tx.I8, tx.BF16, tx.SCALE_ROWCOL), 8.44),
             ((2048, 7168, 7168, tx.F8E4M3, tx.BF16, tx.SCALE_BLOCK128), 41.8)]
    for (M, N, K, a, c, sm), us in cases:
        r = tx.arith_intensity(tx.make_desc(M, N, K, a, c, scale_mode=sm))
        assert r.roofline_us == pytest.approx(us, abs=0.05)


def test_tile_choice():
    big = tx.arith_intensity(tx.make_desc(4096, 4096, 4096, tx.BF16, tx.BF16))
    assert (big.block_m, big.block_n, big.block_k) == (256, 256, 64)
    small = tx.arith_intensity(tx.make_desc(512, 512, 512, tx.F16, tx.F32))
    assert (small.block_m, small.block_n, small.block_k) == (64, 64, 32)
    fixed = tx.arith_intensity(tx.make_desc(512, 512, 512, tx.F16, tx.F32, block=(128, 128, 64)))
    assert (fixed.block_m, fixed.block_n, fixed.block_k) == (128, 128, 64)
    c5 = tx.arith_intensity(tx.make_desc(2048, 7168, 7168, tx.F8E4M3, tx.BF16,
                                         scale_mode=tx.SCALE_BLOCK128))
    assert (c5.block_m, c5.block_n, c5.block_k) == (256, 256, 128)


def test_rejects_bad_desc():
    with pytest.raises(tx.TxError):
        tx.arith_intensity(tx.make_desc(4, 4, 4, 99, tx.F32))
    with pytest.raises(tx.TxError):
        tx.arith_intensity(tx.make_desc(-1, 4, 4, tx.BF16, tx.F32))
