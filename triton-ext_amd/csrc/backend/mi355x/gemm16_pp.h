// bf16/fp16 256x256x64 tile kernel for gfx950 with an eight-wave ping-pong:
// C[M,N] = epilogue(A[M,K] . B[K,N]), all row-major.
//
// Two waves share each SIMD.  Waves 0-3 (group X, output rows 0-127 of the
// tile) and waves 4-7 (group Y, rows 128-255) alternate between a compute
// phase -- the 16 MFMAs of half a K step (2 sub-steps of 16), operands
// already in registers -- and a memory phase -- the 16 LDS reads of their next
// half step.  While one wave of a SIMD issues MFMAs the other issues LDS
// reads and direct-to-LDS loads, so the matrix core is not left waiting on a
// wave that waits on memory; a workgroup barrier separates phases.  With half
// steps h = 2k, 2k+1 of step k:
//
//   phase        X (waves 0-3)            Y (waves 4-7)
//   prologue     read half 0              issue loads of steps 0, 1
//   2h           MFMAs of half h          read half h [h = 2k+1: wait for
//                                         step k+1, issue loads of step k+2]
//   2h+1         read half h+1            MFMAs of half h
//
// LDS holds two stages (step k in stage k % 2, 64 KiB each).  Stage k % 2 is
// last read by Y in phase 4k+2 (half 2k+1), so Y refills it with step k+2 in
// that phase once its own reads have returned; X first reads step k+2 in
// phase 4k+7, and Y waits for those loads (vmcnt(0)) in phase 4k+6.
//
// Each wave owns a 128x64 sub-tile (4x2 blocks of 32x32, 128 fp32
// accumulators) and holds half a K step of operands (8 A and 4 B fragments,
// 48 VGPRs): two waves per SIMD leave 256 registers each.  Staging (layouts, buffer loads into LDS with out-of-range
// zeros, transposed B reads) is gemm16_w4.h's; so is the epilogue layout
// (operand roles swapped: four consecutive columns per register quad).
#pragma once

#include "gemm16_w4.h"

namespace txk {

template <int OP, int EPI> struct Gemm16PP {
  typedef Gemm16W4<OP, EPI, 4> S; // staging partition over 4 waves, helpers
  static constexpr int BM = 256, BN = 256, BK = 64, KS = BK / 16;
  static constexpr int WTM = 128, WTN = 64, FM = WTM / 32, FN = WTN / 32;
  static constexpr int A_BYTES = S::A_BYTES, B_BYTES = S::B_BYTES;
  static constexpr uint32_t STAGE = A_BYTES + B_BYTES;

  static constexpr int HKS = KS / 2; // sub-steps per half step
  struct HalfFrags {
    u32x4 a[HKS][FM];
    i16x8_t b[HKS][FN];
  };

  // Per-lane LDS byte addresses of this wave's fragments in stage 0,
  // sub-step 0.  A: row block i, the lane's row and its chunk after the XOR
  // swizzle; the sub-step only flips address bits 5-6 (chunk bits 1-2), so
  // sub-step ks of stage s is (a[i] + s * STAGE) ^ (ks << 5).  B: column block
  // j; the swizzle term depends on the row within a group of 4 only, so
  // sub-step ks adds ks * 16 rows (an immediate) and the second read + 4 rows.
  struct Bases {
    uint32_t a[FM], b[FN];
  };
  __device__ __forceinline__ static void bases(uint32_t lds0, int wm, int wn, Bases &bs) {
    const int lane = threadIdx.x & 63;
    const int G = lane >> 4, L = lane & 15;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int row = wm * WTM + i * 32 + (lane & 31);
      const int c = lane >> 5; // sub-step 0
      bs.a[i] = lds0 + row * S::RA + ((c ^ ((row ^ (row >> 3)) & (S::NCA - 1))) << 4);
    }
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int n = wn * WTN + j * 32 + 16 * (G & 1) + 4 * (L & 3);
      const int k = 8 * (G >> 1) + (L >> 2); // sub-step 0
      bs.b[j] = lds0 + A_BYTES + k * S::RBB + (((n >> 3) ^ (4 * (k & 3))) << 4) + (n & 7) * 2;
    }
  }

  // Operand fragments of half step `half` (sub-steps 2 half, 2 half + 1) of
  // stage `stage`.
  __device__ __forceinline__ static void read_half(const Bases &bs, int stage, int half,
                                                   HalfFrags &f) {
    typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
    const uint32_t so = (uint32_t)stage * STAGE;
#pragma unroll
    for (int h = 0; h < HKS; ++h) {
      const int ks = half * HKS + h;
#pragma unroll
      for (int i = 0; i < FM; ++i)
        f.a[h][i] = *(const lds_u32x4 *)(uintptr_t)((bs.a[i] + so) ^ ((uint32_t)ks << 5));
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const uint32_t o0 = bs.b[j] + so + ks * 16 * S::RBB;
        const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(uintptr_t)o0);
        const i16x4_t hi =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(uintptr_t)(o0 + 4 * S::RBB));
        f.b[h][j] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
    }
  }

  // The MFMAs of a half step (its first nks sub-steps, 0..2).
  __device__ __forceinline__ static void compute_half(const HalfFrags &f, int nks,
                                                      f32x16_t (&acc)[FM][FN]) {
#pragma unroll
    for (int h = 0; h < HKS; ++h)
      if (h < nks)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[i][j] = S::mma(f.b[h][j], f.a[h][i], acc[i][j]);
  }

  template <bool MASK_MN>
  __device__ __forceinline__ static void run(const GemmArgs &p, int64_t m0, int64_t n0,
                                             uint8_t *smem) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool is_y = wave >= 4;
    const int q = wave & 3; // index within the group
    const int wm = is_y ? 1 : 0, wn = q;
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
    const i32x4_t ra = make_rsrc(p.A, (uint32_t)(((p.M - 1) * p.lda + p.K) * 2));
    const i32x4_t rb = make_rsrc(p.B, (uint32_t)(((p.K - 1) * p.ldb + p.N) * 2));
    // Y's waves issue every load, partitioned as the 4-wave staging does
    // (wave index q): 8 A and 8 B loads of 1 KiB per wave per step.
    typename S::Offsets o;
    if (is_y)
      S::template offsets_q<MASK_MN>(p, m0, n0, q, o);
    auto issue_step = [&](int kt) {
      const uint32_t st = lds0 + (kt & 1) * STAGE;
      if (MASK_MN || kt >= nmain)
        S::template issue_q<true>(p, o, ra, rb, kt, st, q);
      else
        S::template issue_q<false>(p, o, ra, rb, kt, st, q);
    };
    auto barrier = [] { __syncthreads(); };
    // vmcnt(N) with lgkmcnt(0): N = the loads of one step still allowed in flight.
    auto wait_loads = [](bool allow_one_step) {
      if (allow_one_step)
        __builtin_amdgcn_s_waitcnt((16 & 0xf) | ((16 >> 4) << 14) | (0x7 << 4));
      else
        __builtin_amdgcn_s_waitcnt(0x7 << 4);
    };

    auto lgkm_wait = [] { __builtin_amdgcn_s_waitcnt(0x7 << 4 | 0xf | (0x3 << 14)); };
    // Sub-steps of half step h that reach k < K.
    auto half_ks = [&](int h) {
      if ((h >> 1) + 1 < total)
        return HKS;
      const int r = p.last_ks - (h & 1) * HKS;
      return r < 0 ? 0 : (r > HKS ? HKS : r);
    };

    Bases bs;
    bases(lds0, wm, wn, bs);
    HalfFrags f;
    // X and Y run separate loops, each straight-line per half step, with the
    // same number of barriers (the hardware barrier counts waves, not code
    // locations).  Each loop updates the accumulators unconditionally, so
    // they stay in one register set.
    if (total > 0) {
      const int halves = 2 * total;
      if (!is_y) {
        barrier(); // Y's loads of step 0 have landed
        read_half(bs, 0, 0, f);
        lgkm_wait();
        barrier();
        for (int h = 0; h < halves; ++h) {
          __builtin_amdgcn_s_setprio(1);
          compute_half(f, half_ks(h), acc); // phase 2h
          __builtin_amdgcn_s_setprio(0);
          barrier();
          if (h + 1 < halves) { // phase 2h+1
            read_half(bs, ((h + 1) >> 1) & 1, (h + 1) & 1, f);
            lgkm_wait();
          }
          barrier();
        }
      } else {
        issue_step(0);
        if (total > 1)
          issue_step(1);
        wait_loads(total > 1); // step 0 landed
        barrier();
        barrier();
        for (int h = 0; h < halves; ++h) {
          const int kt = h >> 1;
          read_half(bs, kt & 1, h & 1, f); // phase 2h
          lgkm_wait();
          if (h & 1) {
            // After the second half of step kt: step kt+1 must have landed;
            // refill stage kt % 2 with step kt+2.
            __builtin_amdgcn_s_waitcnt(0x7 << 4); // vmcnt(0)
            if (kt + 2 < total)
              issue_step(kt + 2);
          }
          barrier();
          __builtin_amdgcn_s_setprio(1);
          compute_half(f, half_ks(h), acc); // phase 2h+1
          __builtin_amdgcn_s_setprio(0);
          barrier();
        }
      }
    }
    S::template epilogue_tile<MASK_MN, FM, FN, WTM, WTN>(p, m0, n0, wm, wn, acc);
  }
};

template <int OP, int EPI>
__global__ void __launch_bounds__(512, 1) gemm16_pp_kernel(GemmArgs p) {
  typedef Gemm16PP<OP, EPI> G;
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
