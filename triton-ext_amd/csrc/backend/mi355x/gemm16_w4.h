// bf16/fp16 256x256x64 tile kernel for gfx950, four waves of 128x128:
// C[M,N] = epilogue(A[M,K] . B[K,N]), all row-major.
//
// Why four waves.  On gfx950 LDS reads are bounded by instruction issue (about
// one wave-wide read per 4-5 clocks per CU: ds_read_b128 moves 1 KiB,
// ds_read_b64_tr_b16 512 B), and every MFMA operand of this tile passes through
// LDS.  A wave tile of 128x128 (4x4 blocks of 32x32) reuses each A and B
// fragment four times: 12 LDS reads per 16 MFMAs, 192 reads per CU per K step
// against 2048 MFMA clocks per SIMD, where eight 64x128 waves need 320.  The
// 256 fp32 accumulators of a wave live in AGPRs; one wave per SIMD.
//
// Staging is gemm16_dma.h's: direct-to-LDS loads (no VGPR staging) into
// swizzled A [256][64] and B [64][256] tiles, two stages in separate
// __shared__ arrays.  B (N-contiguous) reaches the MFMA through
// ds_read_b64_tr_b16.
//
// Pipeline.  One wave works through the 4 sub-steps (16 of K) of a step:
// while the 16 MFMAs of sub-step s run, the 12 LDS reads of sub-step s+1 are
// in flight.  At the start of the last sub-step every wave has its fragments
// in registers, so a single barrier per step (after s_waitcnt vmcnt(0), which
// also proves the next stage has landed) frees the stage just read; the loads
// of step k+2 then go into it while the MFMAs of step k and k+1 run.
//
// Operand roles are swapped (MFMA A := B columns, MFMA B := A rows), so the
// MFMA result is C^T and lane l holds row m = l % 32 of a 32x32 block at
// columns 8 (r/4) + 4 (l/32) + r%4: four consecutive columns per register
// quad, written as one 8-byte (bf16/fp16) or 16-byte (fp32) store.
//
// K loop in LoopSplit form: k_main_steps unmasked steps, then the masked
// ones (zero-filled past K, the tl.load(mask, other=0) of the reference
// kernel); the last step issues only last_ks of its 4 sub-steps.
#pragma once

#include "gemm16_dma.h"

namespace txk {

typedef short i16x8_t __attribute__((ext_vector_type(8)));

// Raw buffer resource (gfx9 V#): 48-bit base, stride 0, num_records bytes,
// word 3 = 0x00020000 (32-bit data format, no swizzle).  Loads whose offset
// is >= num_records return zeros.  Built from kernel arguments, so uniform.
__device__ __forceinline__ i32x4_t make_rsrc(const void *base, uint32_t bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  i32x4_t r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  r[1] = __builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xffffu));
  r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
  r[3] = 0x00020000;
  return r;
}

template <int OP, int EPI, int NW = 4> struct Gemm16W4 {
  static constexpr int BM = 256, BN = 256, BK = 64;
  // NW = 4: 2x2 waves of 128x128; NW = 8: 2x4 waves of 128x64.
  static constexpr int WM = 2, WN = NW / 2;
  static constexpr int WTM = BM / WM, WTN = BN / WN, FM = WTM / 32, FN = WTN / 32, KS = BK / 16;
  static constexpr int RPS = FM + 2 * FN; // LDS reads per sub-step
  static constexpr int MPS = FM * FN;     // MFMAs per sub-step
  // Staging layouts shared with the DMA tile of the same wave grid.
  typedef Gemm16Dma<OP, BM, BN, BK, WM, WN, 2, EPI> Stage;
  static constexpr int RA = Stage::RA, NCA = Stage::NCA, RBB = Stage::RBB;
  static constexpr int A_BYTES = Stage::A_BYTES, B_BYTES = Stage::B_BYTES;
  static_assert(Stage::NW == NW, "staging partition matches the wave count");
  static_assert(OP == OP_BF16 || OP == OP_F16, "16-bit operands only");

  struct Frags {
    u32x4 a[FM];   // A rows: MFMA B operand
    i16x8_t b[FN]; // B columns (transposed reads): MFMA A operand
  };

  // Fragments of sub-step ks from stage (as, bs).
  __device__ __forceinline__ static void load_frags(const uint8_t *as, const uint8_t *bs, int ks,
                                                    int wm, int wn, Frags &f) {
    const int lane = threadIdx.x & 63;
    const int G = lane >> 4, L = lane & 15;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int row = wm * WTM + i * 32 + (lane & 31);
      const int c = ks * 2 + (lane >> 5);
      f.a[i] = *reinterpret_cast<const u32x4 *>(as + row * RA +
                                                ((c ^ ((row ^ (row >> 3)) & (NCA - 1))) << 4));
    }
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int n = wn * WTN + j * 32 + 16 * (G & 1) + 4 * (L & 3);
      const int k = ks * 16 + 8 * (G >> 1) + (L >> 2), k4 = k + 4;
      const uint32_t off0 = k * RBB + (((n >> 3) ^ (4 * (k & 3))) << 4) + (n & 7) * 2;
      const uint32_t off1 = k4 * RBB + (((n >> 3) ^ (4 * (k4 & 3))) << 4) + (n & 7) * 2;
      const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_i16x4 *)((__attribute__((address_space(3))) uint8_t *)bs + off0));
      const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_i16x4 *)((__attribute__((address_space(3))) uint8_t *)bs + off1));
      f.b[j] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    }
  }

  // Staging.  Buffer loads into LDS (buffer_load_dwordx4 ... lds): every
  // lane has a fixed 32-bit byte offset per load, computed once per tile, and
  // the K step advances through the scalar soffset, so a step's 16 loads
  // cost no VALU.  Chunks outside the matrix get an offset past the buffer's
  // num_records and the hardware returns zeros -- the tl.load(mask, other=0)
  // of the reference kernel -- with no branch:
  //   * rows of A >= M and columns of B >= N: offset kOOB, fixed per tile;
  //   * rows of B >= K: past the end of B already;
  //   * columns of A >= K (masked steps only): offset kOOB for that step.
  // The loads are asm statements (M0 = LDS destination through an operand
  // constraint), so the compiler's wait-count insertion never holds LDS reads
  // of the other stage behind them; the only wait for them is the vmcnt(0)
  // before the next step barrier.
  static constexpr uint32_t kOOB = 0x80000000u; // > num_records (spans < 2 GiB)

  struct Offsets {
    uint32_t a[Stage::A_DMA]; // A: ((m0 + row) * lda + c * 8) * 2, or kOOB
    uint32_t b[Stage::B_DMA]; // B: (k * ldb + n0 + c * 8) * 2, or kOOB
    int32_t ak[Stage::A_DMA]; // A: K index of the chunk within a step
  };

  // Offsets of the loads that staging wave `wave` (0..NW-1) issues.
  template <bool MASK_MN>
  __device__ __forceinline__ static void offsets_q(const GemmArgs &p, int64_t m0, int64_t n0,
                                                   int wave, Offsets &o) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < Stage::A_DMA; ++i) {
      const int j = wave * Stage::A_DMA + i; // 1 KiB block of the A tile
      const int g = j * 64 + lane;           // 16-byte slot in the tile
      const int row = g / NCA, pc = g % NCA;
      const int c = pc ^ ((row ^ (row >> 3)) & (NCA - 1));
      o.ak[i] = c * 8;
      o.a[i] = (MASK_MN && m0 + row >= p.M) ? kOOB : (uint32_t)(((m0 + row) * p.lda + c * 8) * 2);
    }
#pragma unroll
    for (int i = 0; i < Stage::B_DMA; ++i) {
      const int j = wave * Stage::B_DMA + i;
      const int g = j * 64 + lane;
      const int k = g / Stage::NCB, pc = g % Stage::NCB;
      const int c = pc ^ (4 * (k & 3));
      o.b[i] = (MASK_MN && n0 + c * 8 >= p.N) ? kOOB : (uint32_t)((k * p.ldb + n0 + c * 8) * 2);
    }
  }

  __device__ __forceinline__ static void buffer_lds16(uint32_t voff, const i32x4_t &rsrc,
                                                      uint32_t soff, uint32_t lds) {
    asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(rsrc), "s"(soff),
                 "{m0}"(lds)
                 : "memory");
  }

  // Loads of K step kt into the stage at LDS address st.  MASK_K: test A's
  // columns against K (the tail step).  !live: a step past the end (its
  // stage is never read again): every load reads zeros.
  template <bool MASK_K>
  __device__ __forceinline__ static void issue_q(const GemmArgs &p, const Offsets &o,
                                                 const i32x4_t &ra, const i32x4_t &rb, int kt,
                                                 uint32_t st, int wave, bool live = true) {
    const int k0 = kt * BK;
    const uint32_t sa = (uint32_t)k0 * 2u;
    const uint32_t sb = (uint32_t)((int64_t)k0 * p.ldb * 2);
#pragma unroll
    for (int i = 0; i < Stage::A_DMA; ++i) {
      uint32_t v = o.a[i];
      if (MASK_K && (!live || k0 + o.ak[i] >= p.K))
        v = kOOB;
      buffer_lds16(v, ra, sa, st + (wave * Stage::A_DMA + i) * 1024);
    }
#pragma unroll
    for (int i = 0; i < Stage::B_DMA; ++i) {
      uint32_t v = o.b[i];
      if (MASK_K && !live)
        v = kOOB;
      buffer_lds16(v, rb, sb, st + A_BYTES + (wave * Stage::B_DMA + i) * 1024);
    }
  }

  template <bool MASK_MN>
  __device__ __forceinline__ static void offsets(const GemmArgs &p, int64_t m0, int64_t n0,
                                                 Offsets &o) {
    offsets_q<MASK_MN>(p, m0, n0, __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), o);
  }
  template <bool MASK_K>
  __device__ __forceinline__ static void issue(const GemmArgs &p, const Offsets &o,
                                               const i32x4_t &ra, const i32x4_t &rb, int kt,
                                               uint32_t st, bool live = true) {
    issue_q<MASK_K>(p, o, ra, rb, kt, st, __builtin_amdgcn_readfirstlane(threadIdx.x >> 6),
                    live);
  }

  __device__ __forceinline__ static f32x16_t mma(const i16x8_t &bcol, const u32x4 &arow,
                                                 f32x16_t acc) {
    if constexpr (OP == OP_BF16)
      return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, bcol),
                                                     __builtin_bit_cast(bf16x8_t, arow), acc,
                                                     0, 0, 0);
    else
      return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, bcol),
                                                    __builtin_bit_cast(f16x8_t, arow), acc,
                                                    0, 0, 0);
  }

  __device__ __forceinline__ static void mfmas(const Frags &f, f32x16_t (&acc)[FM][FN]) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
        acc[i][j] = mma(f.b[j], f.a[i], acc[i][j]);
  }

  // Scheduling hint for one sub-step: its MPS MFMAs with the RPS LDS reads
  // of the next sub-step spread between them.
  __device__ __forceinline__ static void interleave_reads() {
#pragma unroll
    for (int i = 0; i < MPS; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); // MFMA
      if (i < RPS)
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0); // DS read
    }
  }

  template <bool MASK_MN>
  __device__ __forceinline__ static void run(const GemmArgs &p, int64_t m0, int64_t n0,
                                             uint8_t *smem) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WN, wn = wave % WN;
    f32x16_t acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          acc[i][j][r] = 0.f;

    const int nmain = p.k_main_steps;
    const int total = nmain + p.k_masked_steps;
    const uint32_t lds0 = lds_addr(smem);
    constexpr uint32_t STAGE = A_BYTES + B_BYTES;
    auto stage_ptr = [&](int kt) { return smem + (kt & 1) * STAGE; };
    const i32x4_t ra = make_rsrc(p.A, (uint32_t)(((p.M - 1) * p.lda + p.K) * 2));
    const i32x4_t rb = make_rsrc(p.B, (uint32_t)(((p.K - 1) * p.ldb + p.N) * 2));
    Offsets o;
    offsets<MASK_MN>(p, m0, n0, o);
    // s_waitcnt vmcnt(0) lgkmcnt(0), then the workgroup barrier (with its
    // fences, so no LDS access moves across it).
    auto step_barrier = [] {
      __builtin_amdgcn_s_waitcnt(0x7 << 4); // vmcnt 0, expcnt 7, lgkmcnt 0
      __syncthreads();
    };

    if (total > 0) {
      if (nmain > 0)
        issue<false>(p, o, ra, rb, 0, lds0);
      else
        issue<true>(p, o, ra, rb, 0, lds0);
      step_barrier();
      if (total > 1) {
        if (nmain > 1)
          issue<false>(p, o, ra, rb, 1, lds0 + STAGE);
        else
          issue<true>(p, o, ra, rb, 1, lds0 + STAGE);
      }
      Frags f0, f1;
      load_frags(stage_ptr(0), stage_ptr(0) + A_BYTES, 0, wm, wn, f0);
      // Every step but the last: straight-line, 4 full sub-steps.  The first
      // loop's steps load step kt + 2 unmasked; the second's masked (the K
      // tail) or dead (past the end).
      auto full_step = [&](int kt, auto mask_k) {
        constexpr bool MASK_K = decltype(mask_k)::value;
        const uint8_t *as = stage_ptr(kt), *bs = as + A_BYTES;
        const uint8_t *an = stage_ptr(kt + 1), *bn = an + A_BYTES;
        load_frags(as, bs, 1, wm, wn, f1);
        mfmas(f0, acc);
        interleave_reads();
        load_frags(as, bs, 2, wm, wn, f0);
        mfmas(f1, acc);
        interleave_reads();
        load_frags(as, bs, 3, wm, wn, f1);
        mfmas(f0, acc);
        interleave_reads();
        // Every wave holds sub-step 3's fragments: free this stage, load
        // step kt + 2 into it, read step kt + 1's first fragments.
        step_barrier();
        issue<MASK_K>(p, o, ra, rb, kt + 2, lds0 + (kt & 1) * STAGE, kt + 2 < total);
        load_frags(an, bn, 0, wm, wn, f0);
        mfmas(f1, acc);
        interleave_reads();
      };
      int kt = 0;
      const int unmasked_end = nmain - 2 < total - 1 ? nmain - 2 : total - 1;
      for (; kt < unmasked_end; ++kt)
        full_step(kt, std::integral_constant<bool, false>());
      for (; kt < total - 1; ++kt)
        full_step(kt, std::integral_constant<bool, true>());
      // The last step (the peeled K tail when K % BK != 0): only the
      // sub-steps that reach k < K.
      const uint8_t *as = stage_ptr(kt), *bs = as + A_BYTES;
      const int nks = p.last_ks;
      if (nks > 1)
        load_frags(as, bs, 1, wm, wn, f1);
      mfmas(f0, acc);
      if (nks > 1) {
        if (nks > 2)
          load_frags(as, bs, 2, wm, wn, f0);
        mfmas(f1, acc);
        if (nks > 2) {
          if (nks > 3)
            load_frags(as, bs, 3, wm, wn, f1);
          mfmas(f0, acc);
          if (nks > 3)
            mfmas(f1, acc);
        }
      }
    }

    epilogue_tile<MASK_MN, FM, FN, WTM, WTN>(p, m0, n0, wm, wn, acc);
  }

  // Epilogue of a wave's (FM*32) x (FN*32) sub-tile at (wm, wn): lane l
  // holds, per 32x32 block (i, j) and register quad g, C[row][col .. col+3]
  // with row = m0 + wm*WTM_ + 32 i + l % 32 and col = n0 + wn*WTN_ + 32 j +
  // 8 g + 4 (l / 32).
  template <bool MASK_MN, int FM_, int FN_, int WTM_, int WTN_>
  __device__ __forceinline__ static void epilogue_tile(const GemmArgs &p, int64_t m0,
                                                       int64_t n0, int wm, int wn,
                                                       const f32x16_t (&acc)[FM_][FN_]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < FM_; ++i) {
      const int64_t row = m0 + wm * WTM_ + i * 32 + (lane & 31);
      if (MASK_MN && row >= p.M)
        continue;
#pragma unroll
      for (int j = 0; j < FN_; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int64_t col = n0 + wn * WTN_ + j * 32 + 8 * g + 4 * (lane >> 5);
          if (MASK_MN && col >= p.N) // N % 4 == 0: the quad is all in or all out
            continue;
          const int64_t off = row * p.ldc + col;
          const float v0 = acc[i][j][4 * g], v1 = acc[i][j][4 * g + 1];
          const float v2 = acc[i][j][4 * g + 2], v3 = acc[i][j][4 * g + 3];
          if (EPI == EPI_F32) {
            *reinterpret_cast<float4 *>(reinterpret_cast<float *>(p.C) + off) =
                make_float4(v0, v1, v2, v3);
          } else {
            uint16_t h0, h1, h2, h3;
            if (EPI == EPI_BF16) {
              h0 = f32_to_bf16_rne(v0), h1 = f32_to_bf16_rne(v1);
              h2 = f32_to_bf16_rne(v2), h3 = f32_to_bf16_rne(v3);
            } else {
              h0 = f32_to_f16_rne(v0), h1 = f32_to_f16_rne(v1);
              h2 = f32_to_f16_rne(v2), h3 = f32_to_f16_rne(v3);
            }
            uint2 w;
            w.x = (uint32_t)h0 | ((uint32_t)h1 << 16);
            w.y = (uint32_t)h2 | ((uint32_t)h3 << 16);
            *reinterpret_cast<uint2 *>(reinterpret_cast<uint16_t *>(p.C) + off) = w;
          }
        }
    }
  }
};

template <int OP, int EPI, int NW>
__global__ void __launch_bounds__(NW * 64, 1) gemm16_w4_kernel(GemmArgs p) {
  typedef Gemm16W4<OP, EPI, NW> G;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * (G::A_BYTES + G::B_BYTES)];
  int tm, tn;
  tile_coords(p, tm, tn);
  const int64_t m0 = (int64_t)tm * G::BM, n0 = (int64_t)tn * G::BN;
  if (m0 + G::BM <= p.M && n0 + G::BN <= p.N)
    G::template run<false>(p, m0, n0, smem);
  else
    G::template run<true>(p, m0, n0, smem);
}

} // namespace txk
