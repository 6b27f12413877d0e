// 8-bit operand (fp8 e4m3 / int8) 256x224x128 tile kernel for gfx950:
// C[M,N] = epilogue(A[M,K] . B[K,N]), all row-major.  The same staging,
// MFMAs and block-scale arithmetic as gemm8_w4.h's 256x256 tile, for N a
// multiple of 224 where 256-wide tiles would leave CUs idle (N = 7168:
// 32 tiles of 224 against 28 of 256; with M = 2048, 256 tiles for 256 CUs).
// Measured at that shape it is no faster than 256x256 (its wave layout
// reads B through 28 transposed LDS reads a step against 16), so tile
// selection does not pick it; a caller may ask for it by block size.
//
// Eight waves of 64x112 (4 x 2), each 4 x 7 blocks of 16x16.  A wave keeps
// the A fragments of its 4 row blocks for the whole K step (32 VGPRs) and
// streams B one column block ahead: 7 B columns would not fit beside the
// accumulators (the block-scale FMAs need them in arch VGPRs).  Per column
// block: 4 MFMAs; block-scaled, their partial products get the scale FMA
// during the next column block (the previous step's last column: during
// column 0 of the next step).  The last column block runs after the step
// barrier, replacing each A fragment by the next step's as soon as its MFMA
// is issued.
//
// LDS stage layout: gemm8_w4.h's, B rows still 256 bytes (chunk c of row k
// at c ^ (k & 7)); chunks 14 and 15 (columns 224..255) are never loaded nor
// read.  sb holds the (up to) three 128-column blocks the tile touches.
#pragma once

#include "gemm8_w4.h"

namespace txk {

template <int OP, int EPI> struct Gemm8N224 {
  typedef Gemm8W4<OP, EPI> W; // shared helpers and stage layout
  static constexpr int BM = 256, BN = 224, BNL = W::BN, BK = 128;
  static constexpr int WM = 4, WN = 2, WTM = 64, WTN = 112, FM = 4, FN = 7;
  static constexpr bool SCALED = W::SCALED;
  static constexpr int A_BYTES = W::A_BYTES, SA_OFF = W::SA_OFF, SB_OFF = W::SB_OFF;
  static constexpr uint32_t STAGE = W::STAGE;
  static constexpr int A_DMA = W::A_DMA, B_DMA = W::B_DMA;
  static constexpr uint32_t kOOB = W::kOOB;
  typedef typename W::Acc Acc;
  static_assert(BN % 16 == 0 && BN <= BNL, "tile columns fit the staged rows");

  // Loads of K step kt into stage st, in four parts as gemm8_w4.h (A loads
  // 0,1 + scales / A 2,3 / B 0,1 / B 2,3); B chunks past the tile's 224
  // columns are not loaded.
  template <bool MASK_MN, bool MASK_K, int PART>
  __device__ __forceinline__ static void issue_part(const GemmArgs &p, int64_t m0, int64_t n0,
                                                    const i32x4_t &ra, const i32x4_t &rb,
                                                    const i32x4_t &rsa, const i32x4_t &rsb,
                                                    int kt, uint32_t st, int wave, bool live) {
    const int lane = threadIdx.x & 63;
    const int k0 = kt * BK;
    typedef Gemm16W4<OP_BF16, EPI_F32, 4> L16;
    if (PART < 2) {
#pragma unroll
      for (int i = 2 * PART; i < 2 * PART + 2; ++i) {
        const int j = wave * A_DMA + i;
        const int row = 8 * j + (lane >> 3), pc = lane & 7;
        const int c = pc ^ ((row >> 1) & 7);
        const bool ok = live && (!MASK_MN || m0 + row < p.M) && (!MASK_K || k0 + 16 * c < p.K);
        const uint32_t v = ok ? (uint32_t)(m0 + row) * (uint32_t)p.lda + 16u * c : kOOB;
        L16::buffer_lds16(v, ra, (uint32_t)k0, st + j * 1024);
      }
    } else {
#pragma unroll
      for (int i = 2 * (PART - 2); i < 2 * (PART - 2) + 2; ++i) {
        const int j = wave * B_DMA + i;
        const int k = 4 * j + (lane >> 4), pc = lane & 15;
        const int c = pc ^ (k & 7);
        const bool ok = live && 16 * c < BN && (!MASK_MN || n0 + 16 * c < p.N);
        const uint32_t v = ok ? (uint32_t)k * (uint32_t)p.ldb + (uint32_t)n0 + 16u * c : kOOB;
        L16::buffer_lds16(v, rb, (uint32_t)((int64_t)k0 * p.ldb), st + A_BYTES + j * 1024);
      }
    }
    if (SCALED && PART == 0) {
      if (wave < 4) { // sa[m0 + row][kt], 64 rows per wave
        const int64_t gm = m0 + 64 * wave + lane;
        const uint32_t v = (live && gm < p.M) ? (uint32_t)gm * (uint32_t)(p.sa_ld * 4) : kOOB;
        W::buffer_lds4(v, rsa, (uint32_t)kt * 4, st + SA_OFF + wave * 256);
      }
      if (wave == 0) { // sb[kt][n0/128 + lane], lanes 0..2
        const int64_t nb = (n0 >> 7) + lane;
        const uint32_t v = (live && lane < 3 && nb < p.sb_ld) ? (uint32_t)nb * 4u : kOOB;
        W::buffer_lds4(v, rsb, (uint32_t)(kt * p.sb_ld * 4), st + SB_OFF);
      }
    }
  }

  template <bool MASK_MN>
  __device__ __forceinline__ static void run(const GemmArgs &p, int64_t m0, int64_t n0,
                                             uint8_t *smem) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int G = lane >> 4, L = lane & 15;
    Acc acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          acc[i][j][r] = 0;
    const int nmain = p.k_main_steps;
    const int total = nmain + p.k_masked_steps;
    const uint32_t lds0 = lds_addr(smem);
    // Ranges end at the 16-byte chunk holding each operand's last element.
    const i32x4_t ra = make_rsrc(p.A, (uint32_t)((p.M - 1) * p.lda + ((p.K + 15) & ~15ll)));
    const i32x4_t rb = make_rsrc(p.B, (uint32_t)((p.K - 1) * p.ldb + ((p.N + 15) & ~15ll)));
    i32x4_t rsa = {0, 0, 0, 0}, rsb = {0, 0, 0, 0};
    if (SCALED) {
      rsa = make_rsrc(p.sa, (uint32_t)(p.M * p.sa_ld * 4));
      rsb = make_rsrc(p.sb, (uint32_t)(((p.K + 127) / 128) * p.sb_ld * 4));
    }
    // Per-lane LDS addresses (stage 0): A row block 0 (block i at + 2048 i,
    // the lane's second chunk at ^ 16, as gemm8_w4.h); B: row 32 G + L/2,
    // byte 8 (L % 2) of chunk (7 wn + j) ^ (row & 7).
    const int arow = wm * WTM + L;
    const uint32_t abase = lds0 + arow * BK + (((2 * G) ^ ((arow >> 1) & 7)) << 4);
    const int bk = 32 * G + (L >> 1);
    const uint32_t bbase = lds0 + A_BYTES + bk * BNL + 8 * (L & 1);
    auto read_a = [&](uint32_t so, int i) {
      typedef __attribute__((address_space(3))) i32x4_t lds_i32x4;
      const uint32_t a0 = abase + so + 2048 * i;
      const i32x4_t lo = *(const lds_i32x4 *)(uintptr_t)a0;
      const i32x4_t hi = *(const lds_i32x4 *)(uintptr_t)(a0 ^ 16u);
      i32x8_t r;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        r[t] = lo[t];
        r[4 + t] = hi[t];
      }
      return r;
    };
    auto read_b = [&](uint32_t so, int j) {
      typedef int v2i __attribute__((ext_vector_type(2)));
      typedef __attribute__((address_space(3))) v2i lds_v2i_t;
      const uint32_t b0 = bbase + so + ((uint32_t)((7 * wn + j) ^ (bk & 7)) << 4);
      i32x8_t r;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const v2i v =
            __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i_t *)(uintptr_t)(b0 + q * 8 * BNL));
        r[2 * q] = v.x;
        r[2 * q + 1] = v.y;
      }
      return r;
    };
    typedef __attribute__((address_space(3))) float lds_f32;
    // sa of row block i and sb of column block j, step in stage so.
    auto sa_of = [&](uint32_t so, int i) {
      return *(const lds_f32 *)(uintptr_t)(lds0 + so + SA_OFF + 4 * (wm * WTM + 16 * i + L));
    };
    auto sb_of = [&](uint32_t so, int j) {
      const int nb = (int)(((n0 + wn * WTN + 16 * j) >> 7) - (n0 >> 7));
      return *(const lds_f32 *)(uintptr_t)(lds0 + so + SB_OFF + 4 * nb);
    };
    auto part_of = [&](int kt, auto pc) {
      constexpr int PART = decltype(pc)::value;
      const uint32_t st = lds0 + (kt & 1) * STAGE;
      const bool live = kt < total;
      if (kt >= nmain)
        issue_part<MASK_MN, true, PART>(p, m0, n0, ra, rb, rsa, rsb, kt, st, wave, live);
      else
        issue_part<MASK_MN, false, PART>(p, m0, n0, ra, rb, rsa, rsb, kt, st, wave, live);
    };
    auto step_barrier = [] {
      __builtin_amdgcn_s_waitcnt(0x7 << 4); // vmcnt 0, expcnt 7, lgkmcnt 0
      __syncthreads();
    };
    // Pending partial products of the previous column block, with scales.
    Acc P[FM];
    float sP[FM];
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      P[i] = Acc{0, 0, 0, 0};
      sP[i] = 0.f;
    }
    auto flush = [&](int jd) {
      if constexpr (SCALED) {
#pragma unroll
        for (int i = 0; i < FM; ++i) {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            acc[i][jd][r] = __builtin_fmaf(P[i][r], sP[i], acc[i][jd][r]);
          W::pin(acc[i][jd]);
        }
      }
    };

    if (total > 0) {
      part_of(0, std::integral_constant<int, 0>());
      part_of(0, std::integral_constant<int, 1>());
      part_of(0, std::integral_constant<int, 2>());
      part_of(0, std::integral_constant<int, 3>());
      step_barrier();
      part_of(1, std::integral_constant<int, 0>());
      i32x8_t a[FM];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        a[i] = read_a(0, i);
      i32x8_t bc = read_b(0, 0);
      float sa_c[FM];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        sa_c[i] = SCALED ? sa_of(0, i) : 1.f;
      // One step from stage so; more: a following step exists (issue its
      // remaining loads in column blocks 0..2, the barrier before the last
      // column block, then the next step's A fragments, B column 0, sa).
      auto step = [&](int kt, bool more) {
        const uint32_t so = (kt & 1) * STAGE, sn = ((kt + 1) & 1) * STAGE;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const bool last = j == FN - 1;
          i32x8_t bn;
          if (!last)
            bn = read_b(so, j + 1);
          const float sbj = SCALED ? sb_of(so, j) : 1.f;
          if (more && last) {
            // Every read of this stage is issued; once returned, free it.
            step_barrier();
            part_of(kt + 2, std::integral_constant<int, 0>());
          }
          Acc Q[FM];
#pragma unroll
          for (int i = 0; i < FM; ++i) {
            if constexpr (SCALED)
              Q[i] = W::mma(bc, a[i], Acc{0, 0, 0, 0});
            else
              acc[i][j] = W::mma(bc, a[i], acc[i][j]);
            if (more && last)
              a[i] = read_a(sn, i);
          }
          if (more && j == 0) part_of(kt + 1, std::integral_constant<int, 1>());
          if (more && j == 1) part_of(kt + 1, std::integral_constant<int, 2>());
          if (more && j == 2) part_of(kt + 1, std::integral_constant<int, 3>());
          flush(j == 0 ? FN - 1 : j - 1);
#pragma unroll
          for (int i = 0; i < FM; ++i) {
            P[i] = Q[i];
            sP[i] = sa_c[i] * sbj;
          }
          if (!last)
            bc = bn;
          __builtin_amdgcn_sched_barrier(0);
        }
        if (more) {
          bc = read_b(sn, 0);
#pragma unroll
          for (int i = 0; i < FM; ++i)
            sa_c[i] = SCALED ? sa_of(sn, i) : 1.f;
        }
      };
      for (int kt = 0; kt + 1 < total; ++kt)
        step(kt, true);
      if constexpr (OP == OP_F8) { // fp8 K tail: A's bytes past K (W::mask_k)
#pragma unroll
        for (int i = 0; i < FM; ++i)
          a[i] = W::mask_k(a[i], total - 1, p.K);
      }
      step(total - 1, false);
      flush(FN - 1);
      // Loads of a step past the end may still be writing zeros into LDS.
      __builtin_amdgcn_s_waitcnt(0x7 << 4);
    }
    W::template epilogue_t<MASK_MN, FM, FN, WTM, WTN>(p, m0, n0, wm, wn, acc);
  }
};

template <int OP, int EPI>
__global__ void __launch_bounds__(512, 1) gemm8_n224_kernel(GemmArgs p) {
  typedef Gemm8N224<OP, EPI> G;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * G::STAGE];
  int tm, tn;
  tile_coords(p, tm, tn);
  const int64_t m0 = (int64_t)tm * G::BM, n0 = (int64_t)tn * G::BN;
  if (m0 + G::BM <= p.M && n0 + G::BN <= p.N)
    G::template run<false>(p, m0, n0, smem);
  else
    G::template run<true>(p, m0, n0, smem);
}

} // namespace txk
