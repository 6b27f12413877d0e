// int8 W8A8 small-M dot (decode shape) for gfx950:
//   C[m][n] = bf16((float(sum_k A[m][k] * B[k][n]) * sa[m]) * sb[n])
// with A int8 [M,K] (M <= 16*MT), B int8 [K,N] row-major, int32 accumulation.
//
// The job is a single pass over B (HBM-bound), so the kernel is built around
// streaming B once with wide coalesced loads and keeping every CU busy:
//  * A "batch" is 64 K-rows x 256 N-columns of B (16 KiB) for one wave.  Lane
//    L = j + 16 g loads rows k0 + 16 g + i (i = 0..15) at columns
//    n0 + 16 j .. +15: sixteen 16-byte loads, each wave-wide load reading
//    four 256-byte row segments.
//  * The lane's 16x16 byte block is transposed in registers (byte permutes),
//    giving, for each column c, 16 K-consecutive bytes: exactly the B operand
//    of v_mfma_i32_16x16x64_i8 for K-chunk g, with MFMA column j standing
//    for N column n0 + 16 j + c.  One batch is 16 MFMAs per 16-row tile of A.
//  * Waves of a workgroup take interleaved batches of the workgroup's K
//    range; their int32 partials are summed in LDS.  Workgroups split K
//    (ksplit ways) so that N/256 * ksplit workgroups fill the chip; each
//    writes its int32 partial to the workspace, and the last workgroup of a
//    column strip (atomic arrival counter) adds the partials in split order
//    and applies the epilogue.  Integer addition is exact, so the result is
//    bit-identical to any other summation order.
//  * Arrival counters are never reset: each workgroup adds kMaxSplit/ksplit,
//    so a launch moves every counter by exactly kMaxSplit and the last
//    arrival is the one that brings it to a multiple of kMaxSplit.  The
//    counters must be zero once, when the workspace is created.
#pragma once

#include "gemm_tile.h"

namespace txk {

constexpr int kDecodeBatchK = 64;
constexpr int kDecodeStripN = 256;
constexpr uint32_t kMaxSplit = 64;

struct DecodeArgs {
  const int8_t *A;
  const int8_t *B;
  uint16_t *C;
  const float *sa;
  const float *sb;
  int32_t M, N, K;
  int64_t lda, ldb, ldc;
  int32_t ksplit;           // workgroups per column strip (power of two)
  int32_t batches_per_split;
  int32_t k_main_batches;   // batches with every K row < K (unmasked)
  int32_t *partials;        // [ksplit][M][N] int32
  uint32_t *counters;       // [N / 256] arrival counters
};

__device__ __forceinline__ i32x4_t mfma_i8_16(const u32x4 &a, const u32x4 &b,
                                              i32x4_t acc) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4_t, a),
                                               __builtin_bit_cast(i32x4_t, b),
                                               acc, 0, 0, 0);
}

template <int MT, int WAVES>
__global__ void __launch_bounds__(WAVES * 64)
    decode_i8_kernel(DecodeArgs p) {
  constexpr int MROWS = 16 * MT;
  __shared__ int32_t red[MROWS * kDecodeStripN];
  __shared__ uint32_t last_flag;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int nstrips = (p.N + kDecodeStripN - 1) / kDecodeStripN;
  // Split index varies fastest across consecutive workgroups so that a
  // strip's splits land on different XCDs and CUs.
  const int strip = blockIdx.x / p.ksplit, split = blockIdx.x % p.ksplit;
  const int64_t n0 = (int64_t)strip * kDecodeStripN;
  const int64_t ncol = n0 + 16 * j; // this lane's 16 columns
  const bool col_ok = ncol < p.N;

  for (int i = tid; i < MROWS * kDecodeStripN; i += WAVES * 64)
    red[i] = 0;

  i32x4_t acc[MT][16];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int c = 0; c < 16; ++c)
      acc[t][c] = i32x4_t{0, 0, 0, 0};

  const u32x4 zero = {0u, 0u, 0u, 0u};
  const int b_begin = split * p.batches_per_split;
  int b_end = b_begin + p.batches_per_split;
  const int total_batches = (p.K + kDecodeBatchK - 1) / kDecodeBatchK;
  if (b_end > total_batches)
    b_end = total_batches;

  u32x4 rb[16];
  u32x4 ra[MT];
  auto load = [&](int b) {
    const int64_t k0 = (int64_t)b * kDecodeBatchK;
    const bool mask_k = b >= p.k_main_batches;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int64_t k = k0 + 16 * g + i;
      const bool ok = col_ok && (!mask_k || k < p.K);
      rb[i] = ok ? __builtin_nontemporal_load(
                       reinterpret_cast<const u32x4 *>(p.B + k * p.ldb + ncol))
                 : zero;
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int m = t * 16 + j;
      const int64_t k = k0 + 16 * g;
      const bool ok = m < p.M && (!mask_k || k < p.K);
      ra[t] = ok ? *reinterpret_cast<const u32x4 *>(p.A + m * p.lda + k) : zero;
    }
  };

  int b = b_begin + wave;
  if (b < b_end)
    load(b);
  while (b < b_end) {
    u32x4 tb[16];
    transpose16x16_b8(rb, tb);
    u32x4 a[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t)
      a[t] = ra[t];
    const int nb = b + WAVES;
    if (nb < b_end)
      load(nb); // next batch in flight during this batch's MFMAs
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int c = 0; c < 16; ++c)
        acc[t][c] = mfma_i8_16(a[t], tb[c], acc[t][c]);
    b = nb;
  }
  __syncthreads(); // red[] zeroed

  // acc[t][c] register r of lane (j, g): row t*16 + 4 g + r, column 16 j + c.
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int c = 0; c < 16; ++c)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        atomicAdd(&red[(t * 16 + 4 * g + r) * kDecodeStripN + 16 * j + c],
                  acc[t][c][r]);
  __syncthreads();

  const int nthreads = WAVES * 64;
  if (p.ksplit == 1) {
    for (int i = tid; i < p.M * kDecodeStripN; i += nthreads) {
      const int m = i / kDecodeStripN, n = i % kDecodeStripN;
      if (n0 + n < p.N) {
        const float v = ((float)red[m * kDecodeStripN + n] * p.sa[m]) * p.sb[n0 + n];
        p.C[m * p.ldc + n0 + n] = f32_to_bf16_rne(v);
      }
    }
    return;
  }

  // Publish this split's partial, then count arrivals for the strip.
  int32_t *mine = p.partials + (int64_t)split * p.M * p.N;
  for (int i = tid; i < p.M * kDecodeStripN; i += nthreads) {
    const int m = i / kDecodeStripN, n = i % kDecodeStripN;
    if (n0 + n < p.N)
      mine[(int64_t)m * p.N + n0 + n] = red[m * kDecodeStripN + n];
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const uint32_t inc = kMaxSplit / (uint32_t)p.ksplit;
    const uint32_t old = atomicAdd(&p.counters[strip], inc);
    last_flag = ((old + inc) % kMaxSplit) == 0;
  }
  __syncthreads();
  if (!last_flag)
    return;
  __threadfence();
  for (int i = tid; i < p.M * kDecodeStripN; i += nthreads) {
    const int m = i / kDecodeStripN, n = i % kDecodeStripN;
    const int64_t col = n0 + n;
    if (col < p.N) {
      int32_t s = 0;
      for (int q = 0; q < p.ksplit; ++q) {
        const int32_t *src = p.partials + (int64_t)q * p.M * p.N;
        s += __builtin_nontemporal_load(&src[(int64_t)m * p.N + col]);
      }
      const float v = ((float)s * p.sa[m]) * p.sb[col];
      p.C[m * p.ldc + col] = f32_to_bf16_rne(v);
    }
  }
  (void)nstrips;
}

} // namespace txk
