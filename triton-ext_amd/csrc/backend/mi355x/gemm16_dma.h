// bf16/fp16 tile kernel for gfx950 with direct-to-LDS operand staging and
// LDS transpose reads: C[M,N] = epilogue(A[M,K] . B[K,N]), all row-major.
//
// Staging.  Every operand byte goes global -> LDS through
// global_load_lds_dwordx4: lane l of one wave-wide load writes 16 bytes at
// LDS base + 16 l, so a load fills 1 KiB of LDS and takes no VGPRs.  The LDS
// layouts are swizzled by choosing which global 16-byte chunk each lane
// fetches:
//   A tile [BM][BK], K-contiguous rows of BK*2 bytes; physical chunk
//     pc = c ^ ((row ^ row >> 3) & (chunks - 1)), so the MFMA A reads
//     (32 consecutive rows, one chunk, ds_read_b128) spread over all banks.
//   B tile [BK][BN], N-contiguous rows as in global memory; physical chunk
//     pc = c ^ (BSW * (k & 3)), BSW = 4 for rows of 16 chunks or more
//     (BN >= 128) and 2 for BN = 64, so the transpose reads below, which
//     touch 4 consecutive rows, land on distinct banks.
// Lanes whose chunk lies outside the matrix (K tail, M/N edges) fetch from a
// zero-filled device buffer instead, which is the tl.load(mask, other=0) of the
// reference kernel.  A chunk that crosses K or N (K and N need not fill whole
// 16-byte chunks) is loaded whole: A's elements past K are zeroed in registers
// in the last step, and B's columns past N only reach outputs that are not
// stored.
//
// MFMA operands (v_mfma_f32_32x32x16_{bf16,f16}; lane l holds row/column
// l % 32 and K elements 8 (l / 32) .. +7):
//   A: one ds_read_b128 per 32-row block.
//   B: two ds_read_b64_tr_b16 per 32-column block.  Within each 16-lane group
//      the instruction returns to lane i, element r, the element i % 4 of the
//      64-bit word read by lane 4 r + i / 4; so lane L of group G addresses
//      row k0 + L / 4 at columns n0 + 4 (L % 4) .. +3 and receives column
//      n0 + L, rows k0 .. k0 + 3.  Groups 0/1 cover columns +0/+16 of K rows
//      0..3 (then 4..7), groups 2/3 the same columns for K rows 8..15.
//
// Pipeline: STAGES LDS buffers (separate __shared__ arrays, so the compiler's
// wait-count insertion can tell the buffer being filled from the ones being
// read).  The loads for step k + STAGES - 1 are issued before step k's MFMAs;
// one s_waitcnt vmcnt + barrier per step.
#pragma once

#include "gemm_tile.h"

namespace txk {

typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4;

// Zero-filled source for masked-off chunks (device code refers to it
// directly; it is never written).
__device__ __attribute__((aligned(64))) uint32_t tx_zero_chunk[16];

__device__ __forceinline__ void dma16(const void *src, lds_void *dst) {
  __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
}

// The same with the non-temporal cache policy (gfx940+ cache-policy bit NT,
// value 2): for data read exactly once, which then neither allocates in the
// caches nor forces write-backs of dirty lines to make room.
__device__ __forceinline__ void dma16_stream(const void *src, lds_void *dst) {
  __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 2);
}

// 32-bit LDS address of a __shared__ pointer.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// The direct-to-LDS load as an asm statement (M0 = LDS destination, through
// an operand constraint so the compiler sets it).  The compiler does not see
// it as a write to LDS, so it adds no s_waitcnt vmcnt of its own before LDS
// reads: a caller using it must wait (vmcnt) before reading what it loads.
__device__ __forceinline__ void dma16_asm(const void *src, uint32_t lds) {
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(lds) : "memory");
}

__device__ __forceinline__ u32x4 tr_read_pair(const uint8_t *lds, uint32_t off0,
                                              uint32_t off1) {
  const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_i16x4 *)((__attribute__((address_space(3))) uint8_t *)lds + off0));
  const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_i16x4 *)((__attribute__((address_space(3))) uint8_t *)lds + off1));
  u32x4 r;
  r[0] = (uint16_t)lo[0] | ((uint32_t)(uint16_t)lo[1] << 16);
  r[1] = (uint16_t)lo[2] | ((uint32_t)(uint16_t)lo[3] << 16);
  r[2] = (uint16_t)hi[0] | ((uint32_t)(uint16_t)hi[1] << 16);
  r[3] = (uint16_t)hi[2] | ((uint32_t)(uint16_t)hi[3] << 16);
  return r;
}

template <int OP, int BM, int BN, int BK, int WM, int WN, int STAGES, int EPI>
struct Gemm16Dma {
  typedef OpTraits<OP> T;
  typedef f32x16_t Acc;
  static constexpr int NT = WM * WN * 64;
  static constexpr int NW = WM * WN;
  static constexpr int RA = BK * 2, NCA = RA / 16;   // A row bytes, chunks
  static constexpr int RBB = BN * 2, NCB = RBB / 16; // B row bytes, chunks
  static constexpr int BSW = NCB >= 16 ? 4 : 2;      // B chunk swizzle step
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int FM = WTM / 32, FN = WTN / 32;
  static constexpr int KS = BK / 16;
  static constexpr int A_BYTES = BM * RA, B_BYTES = BK * RBB;
  static constexpr int A_DMA = A_BYTES / 1024 / NW; // wave-wide loads per wave
  static constexpr int B_DMA = B_BYTES / 1024 / NW;
  static constexpr int LDS_BYTES = STAGES * (A_BYTES + B_BYTES);
  static constexpr int DMA_PER_STEP = A_DMA + B_DMA; // vmcnt per K step
  static_assert(STAGES >= 2 && STAGES <= 5, "2..5 stages");
  static_assert(3 * DMA_PER_STEP <= 63, "vmcnt is 6 bits");

  // s_waitcnt vmcnt(N) with the other counters left alone (gfx9 encoding:
  // vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
  template <int N> __device__ __forceinline__ static void vmcnt_wait() {
    __builtin_amdgcn_s_waitcnt((N & 0xf) | ((N >> 4) << 14) | (0x7 << 4) | (0xf << 8));
  }

  static_assert(OP == OP_BF16 || OP == OP_F16, "16-bit operands only");
  static_assert(A_BYTES % (1024 * NW) == 0 && B_BYTES % (1024 * NW) == 0,
                "tiles must split into whole wave-wide loads");
  static_assert(NCB >= 8 && (NCA & (NCA - 1)) == 0, "tile shape");
  static_assert(BK % 16 == 0 && WTM % 32 == 0 && WTN % 32 == 0, "tile shape");

  // Issue the direct-to-LDS loads of K step kt into stage buffer (as, bs).
  template <bool MASK>
  __device__ __forceinline__ static void issue(const GemmArgs &p, int64_t m0, int64_t n0,
                                               int kt, uint8_t *as, uint8_t *bs) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t k0 = (int64_t)kt * BK;
#pragma unroll
    for (int i = 0; i < A_DMA; ++i) {
      const int j = wave * A_DMA + i;       // 1 KiB block of the A tile
      const int g = j * 64 + lane;          // 16-byte slot in the tile
      const int row = g / NCA, pc = g % NCA;
      const int c = pc ^ ((row ^ (row >> 3)) & (NCA - 1));
      const int64_t gm = m0 + row, gk = k0 + c * 8;
      const void *src = p.A + (gm * p.lda + gk) * 2;
      if (MASK && (gm >= p.M || gk >= p.K))
        src = tx_zero_chunk;
      dma16(src, (lds_void *)(as + j * 1024));
    }
#pragma unroll
    for (int i = 0; i < B_DMA; ++i) {
      const int j = wave * B_DMA + i;
      const int g = j * 64 + lane;
      const int k = g / NCB, pc = g % NCB;
      const int c = pc ^ (BSW * (k & 3));
      const int64_t gk = k0 + k, gn = n0 + c * 8;
      const void *src = p.B + (gk * p.ldb + gn) * 2;
      if (MASK && (gk >= p.K || gn >= p.N))
        src = tx_zero_chunk;
      dma16(src, (lds_void *)(bs + j * 1024));
    }
  }

  // MFMA sub-steps [0, nks) of one staged K step.  krem: K minus the step's
  // first K index; elements at or past it (the last step only: a 16-byte
  // chunk that crosses K is loaded whole) are zeroed in A's fragments, whose
  // lane l holds K values 8 c .. 8 c + 7 of the step, c = 2 ks + l / 32.
  // B's rows past K come from the zero chunk.
  __device__ __forceinline__ static void
  compute(const uint8_t *as, const uint8_t *bs, int nks, Acc (&acc)[FM][FN], int64_t krem = BK) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int G = lane >> 4, L = lane & 15;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (ks < nks) {
        u32x4 a[FM], b[FN];
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          const int row = wm * WTM + i * 32 + (lane & 31);
          const int c = ks * 2 + (lane >> 5);
          a[i] = *reinterpret_cast<const u32x4 *>(as + row * RA +
                                                  ((c ^ ((row ^ (row >> 3)) & (NCA - 1))) << 4));
        }
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int n = wn * WTN + j * 32 + 16 * (G & 1) + 4 * (L & 3);
          const int k = ks * 16 + 8 * (G >> 1) + (L >> 2);
          const uint32_t off0 = k * RBB + (((n >> 3) ^ (BSW * (k & 3))) << 4) + (n & 7) * 2;
          const int k4 = k + 4;
          const uint32_t off1 = k4 * RBB + (((n >> 3) ^ (BSW * (k4 & 3))) << 4) + (n & 7) * 2;
          b[j] = tr_read_pair(bs, off0, off1);
        }
        const int64_t rem = krem - (ks * 16 + 8 * (lane >> 5));
        if (rem < 8) {
          u32x4 m;
#pragma unroll
          for (int w = 0; w < 4; ++w)
            m[w] = rem >= 2 * w + 2 ? 0xffffffffu : rem == 2 * w + 1 ? 0x0000ffffu : 0u;
#pragma unroll
          for (int i = 0; i < FM; ++i)
            a[i] &= m;
        }
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j) {
            Frag<1> fa, fb;
            fa.v[0] = a[i];
            fb.v[0] = b[j];
            acc[i][j] = mfma(T(), fa, fb, acc[i][j]);
          }
      }
    }
  }

  template <bool MASK_MN>
  __device__ __forceinline__ static void run(const GemmArgs &p, int64_t m0, int64_t n0,
                                             uint8_t *const (&as)[STAGES],
                                             uint8_t *const (&bs)[STAGES]) {
    static_assert(STAGES >= 2, "");
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WN, wn = wave % WN;
    Acc acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          acc[i][j][r] = 0.f;

    const int nmain = p.k_main_steps;
    const int total = nmain + p.k_masked_steps;
    auto issue_step = [&](int kt, uint8_t *a_dst, uint8_t *b_dst) {
      if (MASK_MN || kt >= nmain)
        issue<true>(p, m0, n0, kt, a_dst, b_dst);
      else
        issue<false>(p, m0, n0, kt, a_dst, b_dst);
    };
    // Wait until this wave's loads for step kt have landed -- the loads of
    // the `newer` steps issued after it may stay in flight -- then barrier so
    // every wave's loads for step kt are visible.
    auto step_barrier = [](int newer) {
      if (newer <= 0)
        vmcnt_wait<0>();
      else if (newer == 1)
        vmcnt_wait<DMA_PER_STEP>();
      else if (newer == 2)
        vmcnt_wait<2 * DMA_PER_STEP>();
      else
        vmcnt_wait<3 * DMA_PER_STEP>();
      __syncthreads();
    };
    if (total > 0) {
      // Prologue: fill STAGES-1 buffers.
#pragma unroll
      for (int s = 0; s < STAGES - 1; ++s)
        if (s < total)
          issue_step(s, as[s], bs[s]);
      // Every step but the last, unrolled by STAGES so buffer indices are static.
      for (int kt0 = 0; kt0 < total - 1; kt0 += STAGES) {
#pragma unroll
        for (int s = 0; s < STAGES; ++s) {
          const int kt = kt0 + s;
          if (kt < total - 1) {
            const int newer = total - 1 - kt < STAGES - 2 ? total - 1 - kt : STAGES - 2;
            step_barrier(newer);
            const int kn = kt + STAGES - 1; // step whose loads go out now
            const int sn = (s + STAGES - 1) % STAGES;
            if (kn < total)
              issue_step(kn, as[sn], bs[sn]);
            compute(as[s], bs[s], KS, acc);
          }
        }
      }
      // The last step (the peeled K tail when K % BK != 0): only the MFMA
      // sub-steps that reach k < K.
      step_barrier(0);
      const int sl = (total - 1) % STAGES;
#pragma unroll
      for (int s = 0; s < STAGES; ++s)
        if (s == sl)
          compute(as[s], bs[s], p.last_ks, acc, p.K - (int64_t)(total - 1) * BK);
    }

    epilogue<MASK_MN>(p, m0, n0, acc);
  }

  // Epilogue: accumulator register r of lane l in a 32x32 block holds row
  // 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32.
  template <bool MASK_MN>
  __device__ __forceinline__ static void epilogue(const GemmArgs &p, int64_t m0, int64_t n0,
                                                  const Acc (&acc)[FM][FN]) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WN, wn = wave % WN;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int64_t col = n0 + wn * WTN + j * 32 + (lane & 31);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t row = m0 + wm * WTM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          if (MASK_MN && (row >= p.M || col >= p.N))
            continue;
          const int64_t off = row * p.ldc + col;
          if (EPI == EPI_F32) {
            float *c = reinterpret_cast<float *>(p.C) + off;
            *c = p.accumulate ? *c + acc[i][j][r] : acc[i][j][r];
          }
          else if (EPI == EPI_BF16)
            reinterpret_cast<uint16_t *>(p.C)[off] = f32_to_bf16_rne(acc[i][j][r]);
          else
            reinterpret_cast<uint16_t *>(p.C)[off] = f32_to_f16_rne(acc[i][j][r]);
        }
      }
  }
};

template <int OP, int BM, int BN, int BK, int WM, int WN, int STAGES, int EPI>
__global__ void __launch_bounds__(WM * WN * 64, 1)
    gemm16_dma_kernel(GemmArgs p) {
  typedef Gemm16Dma<OP, BM, BN, BK, WM, WN, STAGES, EPI> G;
  // One __shared__ array per stage and operand (distinct objects, so the
  // compiler's alias analysis separates the buffer being filled from the one
  // being read).  Arrays of unused stages are never referenced.
  __shared__ __attribute__((aligned(1024))) uint8_t a0[G::A_BYTES], b0[G::B_BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t a1[G::A_BYTES], b1[G::B_BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t a2[STAGES > 2 ? G::A_BYTES : 1];
  __shared__ __attribute__((aligned(1024))) uint8_t b2[STAGES > 2 ? G::B_BYTES : 1];
  __shared__ __attribute__((aligned(1024))) uint8_t a3[STAGES > 3 ? G::A_BYTES : 1];
  __shared__ __attribute__((aligned(1024))) uint8_t b3[STAGES > 3 ? G::B_BYTES : 1];
  __shared__ __attribute__((aligned(1024))) uint8_t a4[STAGES > 4 ? G::A_BYTES : 1];
  __shared__ __attribute__((aligned(1024))) uint8_t b4[STAGES > 4 ? G::B_BYTES : 1];
  uint8_t *const all_a[5] = {a0, a1, a2, a3, a4};
  uint8_t *const all_b[5] = {b0, b1, b2, b3, b4};
  uint8_t *as[STAGES], *bs[STAGES];
#pragma unroll
  for (int s = 0; s < STAGES; ++s) {
    as[s] = all_a[s];
    bs[s] = all_b[s];
  }
  int tm, tn;
  tile_coords(p, tm, tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  if (m0 + BM <= p.M && n0 + BN <= p.N)
    G::template run<false>(p, m0, n0, (uint8_t *const(&)[STAGES])as, (uint8_t *const(&)[STAGES])bs);
  else
    G::template run<true>(p, m0, n0, (uint8_t *const(&)[STAGES])as, (uint8_t *const(&)[STAGES])bs);
}

} // namespace txk
