// bf16/fp16 tile kernel for gfx950 with register-staged operands and LDS
// transpose reads: C[M,N] = epilogue(A[M,K] . B[K,N]), all row-major.
//
// Same LDS layouts and MFMA inner loop as gemm16_dma.h (Gemm16Dma::compute);
// only the global -> LDS path differs.  Each thread owns the same 16-byte LDS
// slots a wave-wide direct-to-LDS load would fill (slot j*64 + lane of block
// j), fetches the swizzled global chunk for each into VGPRs with
// global_load_dwordx4 and later stores it with ds_write_b128, so every LDS
// write of a wave is one contiguous 1 KiB run.
//
// Pipeline: two LDS buffers and RSTAGES register buffers.  With RSTAGES = 2
// the loads of step k + 3 are issued during step k and written to LDS at the
// end of step k + 2: two full steps of MFMA work cover each load's latency
// (the direct-to-LDS kernel covers one).
#pragma once

#include "gemm16_dma.h"

namespace txk {

template <int OP, int BM, int BN, int BK, int WM, int WN, int RSTAGES, int EPI>
struct Gemm16Reg {
  typedef Gemm16Dma<OP, BM, BN, BK, WM, WN, 2, EPI> D; // layouts + compute
  typedef typename D::Acc Acc;
  static constexpr int NT = D::NT, NW = D::NW;
  static constexpr int NCA = D::NCA, NCB = D::NCB;
  static constexpr int FM = D::FM, FN = D::FN, WTM = D::WTM, WTN = D::WTN;
  static constexpr int KS = D::KS;
  static constexpr int A_BYTES = D::A_BYTES, B_BYTES = D::B_BYTES;
  static constexpr int A_LD = D::A_DMA, B_LD = D::B_DMA; // 16-byte loads per thread
  static constexpr int LD = A_LD + B_LD;
  static_assert(RSTAGES == 1 || RSTAGES == 2, "one or two register stages");
  static_assert(RSTAGES * LD <= 63, "vmcnt is 6 bits");

  struct Regs {
    u32x4 v[LD];
  };

  template <int N> __device__ __forceinline__ static void vmcnt_wait() {
    __builtin_amdgcn_s_waitcnt((N & 0xf) | ((N >> 4) << 14) | (0x7 << 4) | (0xf << 8));
  }

  template <bool MASK>
  __device__ __forceinline__ static void load(const GemmArgs &p, int64_t m0, int64_t n0,
                                              int kt, Regs &r) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t k0 = (int64_t)kt * BK;
    const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      const int g = (wave * A_LD + i) * 64 + lane;
      const int row = g / NCA, pc = g % NCA;
      const int c = pc ^ ((row ^ (row >> 3)) & (NCA - 1));
      const int64_t gm = m0 + row, gk = k0 + c * 8;
      const bool ok = !MASK || (gm < p.M && gk < p.K);
      r.v[i] = ok ? *reinterpret_cast<const u32x4 *>(p.A + (gm * p.lda + gk) * 2) : zero;
    }
#pragma unroll
    for (int i = 0; i < B_LD; ++i) {
      const int g = (wave * B_LD + i) * 64 + lane;
      const int k = g / NCB, pc = g % NCB;
      const int c = pc ^ (4 * (k & 3));
      const int64_t gk = k0 + k, gn = n0 + c * 8;
      const bool ok = !MASK || (gk < p.K && gn < p.N);
      r.v[A_LD + i] = ok ? *reinterpret_cast<const u32x4 *>(p.B + (gk * p.ldb + gn) * 2) : zero;
    }
  }

  __device__ __forceinline__ static void write(const Regs &r, uint8_t *as, uint8_t *bs) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int i = 0; i < A_LD; ++i)
      *reinterpret_cast<u32x4 *>(as + ((wave * A_LD + i) * 64 + lane) * 16) = r.v[i];
#pragma unroll
    for (int i = 0; i < B_LD; ++i)
      *reinterpret_cast<u32x4 *>(bs + ((wave * B_LD + i) * 64 + lane) * 16) = r.v[A_LD + i];
  }

  template <bool MASK_MN>
  __device__ __forceinline__ static void run(const GemmArgs &p, int64_t m0, int64_t n0,
                                             uint8_t *as0, uint8_t *bs0, uint8_t *as1,
                                             uint8_t *bs1) {
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
    auto ld = [&](int kt, Regs &r) {
      if (MASK_MN || kt >= nmain)
        load<true>(p, m0, n0, kt, r);
      else
        load<false>(p, m0, n0, kt, r);
    };
    if (total > 0) {
      Regs r0, r1;
      // Prologue: step 0 into LDS buffer 0; steps 1 (.. 2) in flight.
      ld(0, r0);
      if (RSTAGES == 2 && total > 1)
        ld(1, r1);
      if (RSTAGES == 2 && total > 1)
        vmcnt_wait<LD>();
      else
        vmcnt_wait<0>();
      write(r0, as0, bs0);
      if (RSTAGES == 1) {
        if (total > 1)
          ld(1, r0);
      } else {
        if (total > 2)
          ld(2, r0);
      }
      __syncthreads();
      // Steady state, unrolled by two so LDS and register buffers are static.
      // Iteration kt: compute buffer kt%2, then write step kt+1 (held in the
      // register buffer loaded longest ago) to the other LDS buffer and
      // reuse that register buffer for step kt+1+RSTAGES.
      auto iter = [&](int kt, uint8_t *ca, uint8_t *cb, uint8_t *na, uint8_t *nb,
                      Regs &rn, Regs &rother) {
        const bool last = kt == total - 1;
        D::compute(ca, cb, last ? p.last_ks : KS, acc);
        if (!last) {
          // step kt+1 lives in rn; with two register stages, step kt+2 (in
          // rother) may still be in flight.
          if (RSTAGES == 2 && kt + 2 < total)
            vmcnt_wait<LD>();
          else
            vmcnt_wait<0>();
          write(rn, na, nb);
          if (kt + 1 + RSTAGES < total)
            ld(kt + 1 + RSTAGES, rn);
          __syncthreads();
        }
        (void)rother;
      };
      for (int kt = 0; kt < total; kt += 2) {
        if (RSTAGES == 1) {
          iter(kt, as0, bs0, as1, bs1, r0, r1);
          if (kt + 1 < total)
            iter(kt + 1, as1, bs1, as0, bs0, r0, r1);
        } else {
          iter(kt, as0, bs0, as1, bs1, r1, r0);
          if (kt + 1 < total)
            iter(kt + 1, as1, bs1, as0, bs0, r0, r1);
        }
      }
    }
    D::template epilogue<MASK_MN>(p, m0, n0, acc);
  }
};

template <int OP, int BM, int BN, int BK, int WM, int WN, int RSTAGES, int EPI>
__global__ void __launch_bounds__(WM * WN * 64, 1)
    gemm16_reg_kernel(GemmArgs p) {
  typedef Gemm16Reg<OP, BM, BN, BK, WM, WN, RSTAGES, EPI> G;
  __shared__ __attribute__((aligned(1024))) uint8_t a0[G::A_BYTES], b0[G::B_BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t a1[G::A_BYTES], b1[G::B_BYTES];
  int tm, tn;
  tile_coords(p, tm, tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  if (m0 + BM <= p.M && n0 + BN <= p.N)
    G::template run<false>(p, m0, n0, a0, b0, a1, b1);
  else
    G::template run<true>(p, m0, n0, a0, b0, a1, b1);
}

} // namespace txk
