// Fused attention forward for gfx950: the forward of the fused-attention
// tutorial (R:pass/LoopSplit/06-fused-attention.py:44-93, :181-239), fp16
// (the tutorial's type) or bf16 q/k/v/o, HEAD_DIM 16, 32, 64, 128 or 256,
// fp32 softmax statistics and accumulator.  HEAD_DIM 16 runs in the layout
// of 32: its K/V chunks past dim 16 load as zeros (out-of-range buffer
// offsets), Q's dims past 16 are zero and O's are not stored, so S and P V
// are unchanged.
//
// A workgroup owns BM query rows of one (z, h), one wave per 32 rows; BM x
// BN is any of the tutorial's autotuned blocks (64 or 128 by 32 or 64, 128 x
// 64 by default).  Per K/V block of BN keys:
//   S^T = K . Q^T    32x32x16 f16 MFMAs, A := K rows (LDS), B := Q rows (held
//                    in registers for the whole loop), so lane l holds query
//                    row m = l%32 and keys n = 8 (r/4) + 4 (l/32) + r%4 of each
//                    32-key block: a row's statistics need one exchange with
//                    lane l ^ 32;
//   softmax          the tutorial's arithmetic per element (scale, mask,
//                    running max, exp2, running sum);
//   O^T += V^T . P^T A := V columns (LDS transpose reads), B := P straight from
//                    the S^T registers: MFMA slot s of lane group g is key
//                    16 c + 8 (s/4) + 4 g + s%4, so V's rows are read in that
//                    order and no value crosses lanes.
// Staging: K and V blocks (BN x HEAD_DIM x 2 bytes each) reach LDS by direct-to-LDS
// buffer loads into two slots each, one barrier per block; loads run a block
// ahead under the math (the pipeline is described at the kernel).  LDS
// layouts (rows of 2 HEAD_DIM bytes, 16-byte chunk c of row r stored at):
//   K: c ^ ((r >> 2) & 3) (64-byte rows), c ^ ((r >> 1) & 7) (128-byte
//      rows), c ^ (r & 15) (256- and 512-byte rows): the 16 rows a
//      ds_read_b128 pass touches hit 16 different bank groups;
//   V: c (64-byte rows), c ^ (4 ((r >> 1) & 1)) (128-byte rows), c ^ (4 (r &
//      3)) (256- and 512-byte rows): the 4 rows x 64 bytes a
//      ds_read_b64_tr_b16 pass touches cover all 64 banks once.
// The K/V loop runs in LoopSplit form: keys [0, causal_start) unmasked, then
// the on-band blocks [causal_start, causal_start + BM) masked; causal_start =
// start_m * BM, or N_CTX without the causal mask.  Blocks past the diagonal
// are skipped (their p is exactly 0 and alpha exactly 1).
#pragma once

#include "gemm16_w4.h"

namespace txk {

struct AttnArgs {
  const void *Q, *K, *V; // fp16 / bf16, or e5m2 bytes (attn_fwd8.h)
  void *O;
  float *M;
  int64_t q_sz, q_sh, q_sm;
  int64_t k_sz, k_sh, k_sm;
  int64_t v_sz, v_sh, v_sm;
  int64_t o_sz, o_sh, o_sm;
  int32_t H, N_CTX;
  float qk_scale;
};

// BM_ x BN_: the tutorial's autotuned block space, BLOCK_M in {64, 128} (one
// wave per 32 query rows) and BLOCK_N in {32, 64}.
template <int HD, bool BF, int BM_ = 128, int BN_ = 64> struct AttnFwd {
  // D: the head dim of the layout (32 for HEAD_DIM 16); DR: the real one
  static constexpr int BM = BM_, BN = BN_, D = HD < 32 ? 32 : HD, DR = HD, NW = BM_ / 32,
                       ESZ = 2;
  static constexpr int ROW = D * 2;            // bytes per K/V row
  static constexpr int TILE = BN * ROW;        // 2 .. 32 KiB
  // LW: the waves that stage a K/V block, all of them unless the block holds
  // fewer 1 KiB loads than there are waves (2 KiB for 4 waves at head dims
  // 16 and 32 with 128 x 32 blocks: waves 0 and 1 load, 2 and 3 only wait
  // at the barriers that publish every block).
  static constexpr int LW = TILE / 1024 < NW ? TILE / 1024 : NW;
  static constexpr int DMA = TILE / 1024 / LW; // 16-byte loads per lane per tile: 1 .. 8
  static constexpr int CPR = ROW / 16;         // 16-byte chunks per row: 8 / 16
  static constexpr uint32_t kOOB = 0x80000000u;
  static_assert(D == 32 || D == 64 || D == 128 || D == 256, "head dims 16 .. 256");
  static_assert(DR == D || (DR == 16 && D == 32), "head dim 16 in the layout of 32");
  static_assert((BM == 64 || BM == 128) && (BN == 32 || BN == 64), "the tutorial's blocks");
  static_assert(LW >= 1 && DMA >= 1 && DMA * LW * 1024 == TILE, "whole 1 KiB loads per wave");
  // Fragment reads issued together in qk / pv: every one at head dims up to
  // 128, in groups of 8 at 256 (all 32 would take 128 VGPRs).
  static constexpr int KGRP = D / 16 < 8 ? D / 16 : 8;
  // 16-bit element vectors; BF: bf16, else fp16
  typedef typename std::conditional<BF, __bf16, _Float16>::type elt;
  typedef elt h8 __attribute__((ext_vector_type(8)));
  typedef elt h4 __attribute__((ext_vector_type(4)));
  typedef float f16v __attribute__((ext_vector_type(16)));

  __device__ __forceinline__ static f16v mfma(const h8 &a, const h8 &b, const f16v &c) {
    if constexpr (BF)
      return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    else
      return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  // swizzles of the 16-byte chunk index (see the layouts above)
  __device__ __forceinline__ static int kswz(int r) {
    return D == 32 ? (r >> 2) & 3 : D == 64 ? (r >> 1) & 7 : r & 15;
  }
  __device__ __forceinline__ static int vswz(int r) {
    return D == 32 ? 0 : D == 64 ? 4 * ((r >> 1) & 1) : 4 * (r & 3);
  }

  __device__ __forceinline__ static void dma16(uint32_t voff, const i32x4_t &rsrc, uint32_t soff,
                                               uint32_t lds) {
    asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(rsrc), "s"(soff),
                 "{m0}"(lds)
                 : "memory");
  }

  // Per-lane source byte offsets of the wave's DMA loads (relative to the
  // block's first row): load u of wave w fills 1 KiB of LDS, rows
  // (64/CPR) (DMA w + u) .., lane i row .. + i/CPR at chunk position i%CPR,
  // which holds chunk i%CPR ^ swizzle(row) of the source row (V_SWZ: V's
  // layout, else K's).  Chunks past the real head dim take kOOB (zeros).
  template <bool V_SWZ>
  __device__ __forceinline__ static void dma_offsets(int wave, int64_t sm, uint32_t (&o)[DMA]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int u = 0; u < DMA; ++u) {
      const int row = (64 / CPR) * (DMA * wave + u) + lane / CPR, pos = lane % CPR;
      const int c = pos ^ (V_SWZ ? vswz(row) : kswz(row));
      o[u] = 8 * c >= DR ? kOOB : (uint32_t)((row * sm + c * 8) * 2);
    }
  }

  // Loads of K block j into K slot `slot` (V block j into V slot `slot`);
  // none from waves past LW (`wave` is wave-uniform).
  __device__ __forceinline__ static void issue(const i32x4_t &rsrc, const uint32_t (&off)[DMA],
                                               int64_t sm, int j, uint32_t slot_lds, int wave) {
    if (LW < NW && wave >= LW)
      return;
#pragma unroll
    for (int u = 0; u < DMA; ++u)
      dma16(off[u], rsrc, (uint32_t)((int64_t)j * BN * sm * 2), slot_lds + (DMA * wave + u) * 1024);
  }

  // Per-lane LDS addresses (slot 0) of the fragment reads.  Every other
  // fragment is one of these plus a constant, which the reads take as their
  // immediate offset:
  //   K, key block b, dim chunk c: lane l reads key 32 b + l%32, dims
  //     16 c + 8 (l/32) .. +7 at chunk (2c + l/32) ^ ((key >> 1) & 7); the
  //     swizzle does not depend on b, so kb[c] + 32 b ROW;
  //   V^T, dim block bd, key chunk c: two transposed reads (keys 16 c +
  //     4 (l/32) + (L/4) and +8 for lane group l/16 and L = l%16); the
  //     swizzle term depends on key bits 0-1 only, which L fixes, so
  //     vb[bd] + 16 c ROW (+ 8 ROW for the second read).
  struct Bases {
    uint32_t k[D / 16], v[D / 32];
  };
  __device__ __forceinline__ static void bases(uint32_t k_lds, uint32_t v_lds, Bases &bs) {
    const int lane = threadIdx.x & 63;
    const int G = lane >> 4, L = lane & 15, r = lane & 31;
#pragma unroll
    for (int c = 0; c < D / 16; ++c)
      bs.k[c] = k_lds + r * ROW + (((2 * c + (lane >> 5)) ^ kswz(r)) << 4);
#pragma unroll
    for (int bd = 0; bd < D / 32; ++bd) {
      const int d = 32 * bd + 16 * (G & 1) + 4 * (L & 3);
      const int k0 = 4 * (G >> 1) + (L >> 2);
      bs.v[bd] = v_lds + k0 * ROW + (((d >> 3) ^ vswz(k0)) << 4) + (d & 7) * 2;
    }
  }

  template <int SLOT>
  __device__ __forceinline__ static h8 read_k(const Bases &bs, int b, int c) {
    typedef __attribute__((address_space(3))) h8 lds_h8;
    return *(const lds_h8 *)(uintptr_t)(bs.k[c] + SLOT * TILE + b * 32 * ROW);
  }
  template <int SLOT>
  __device__ __forceinline__ static h8 read_v(const Bases &bs, int bd, int c) {
    const uint32_t a = bs.v[bd] + SLOT * TILE + c * 16 * ROW;
    const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(uintptr_t)a);
    const i16x4_t hi =
        __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(uintptr_t)(a + 8 * ROW));
    return __builtin_bit_cast(h8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  }

  // Row statistics across the lane pair (l, l ^ 32): v_permlane32_swap hands
  // each lane both halves' values ([lo, lo] and [hi, hi]) without an LDS
  // round trip, and both lanes form the same result.
  __device__ __forceinline__ static float xmax(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                    false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  }
  __device__ __forceinline__ static float xsum(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                    false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }

  // S^T block of the keys in K slot SLOT: lane holds query row l%32.
  template <int SLOT>
  __device__ __forceinline__ static void qk(const Bases &bs, const h8 (&qf)[D / 16],
                                            f16v (&s)[BN / 32]) {
#pragma unroll
    for (int b = 0; b < BN / 32; ++b)
      s[b] = f16v{};
#pragma unroll
    for (int c0 = 0; c0 < D / 16; c0 += KGRP) {
      h8 kf[BN / 32][KGRP];
#pragma unroll
      for (int b = 0; b < BN / 32; ++b)
#pragma unroll
        for (int c = 0; c < KGRP; ++c)
          kf[b][c] = read_k<SLOT>(bs, b, c0 + c);
#pragma unroll
      for (int b = 0; b < BN / 32; ++b)
#pragma unroll
        for (int c = 0; c < KGRP; ++c)
          s[b] = mfma(kf[b][c], qf[c0 + c], s[b]);
    }
  }

  // Softmax of one block (the tutorial's arithmetic) for the lane's query
  // row m, keys n0 + 8 (r/4) + 4 g + r%4 of each 32-key block: updates m_i and
  // l_i, rescales acc by alpha and returns P as MFMA B operands (key chunk c
  // = registers 8 (c%2) .. +7 of key block c/2).  MASK: on-band form.
  template <bool MASK>
  __device__ __forceinline__ static void softmax(f16v (&s)[BN / 32], int n0, int m,
                                                 float qk_scale, f16v (&acc)[D / 32],
                                                 float &m_i, float &l_i, h8 (&pf)[BN / 16]) {
    const int g = (threadIdx.x & 63) >> 5;
    float m_ij;
    if constexpr (MASK) {
      // qk = qk * qk_scale + where(m >= n, 0, -1e6); m_ij = max(m_i, rowmax(qk))
      float mx = -INFINITY;
#pragma unroll
      for (int b = 0; b < BN / 32; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
#pragma clang fp contract(off)
          const int n = n0 + 32 * b + 8 * (r / 4) + 4 * g + (r % 4);
          float t = s[b][r] * qk_scale;
          t = t + (m >= n ? 0.0f : -1.0e6f);
          s[b][r] = t;
          mx = fmaxf(mx, t);
        }
      m_ij = fmaxf(m_i, xmax(mx));
#pragma unroll
      for (int b = 0; b < BN / 32; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          s[b][r] = __builtin_amdgcn_exp2f(s[b][r] - m_ij);
    } else {
      // m_ij = max(m_i, rowmax(qk) * qk_scale); qk = qk * qk_scale - m_ij
      float mx = -INFINITY;
#pragma unroll
      for (int b = 0; b < BN / 32; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          mx = fmaxf(mx, s[b][r]);
      m_ij = fmaxf(m_i, xmax(mx) * qk_scale);
#pragma unroll
      for (int b = 0; b < BN / 32; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          s[b][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[b][r], qk_scale, -m_ij));
    }
    float l_ij = 0.f;
#pragma unroll
    for (int b = 0; b < BN / 32; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        l_ij += s[b][r];
    l_ij = xsum(l_ij);
    const float alpha = __builtin_amdgcn_exp2f(m_i - m_ij);
    l_i = l_i * alpha + l_ij;
    m_i = m_ij;
#pragma unroll
    for (int c = 0; c < BN / 16; ++c)
#pragma unroll
      for (int t = 0; t < 8; ++t)
        pf[c][t] = (elt)s[c / 2][8 * (c % 2) + t];
#pragma unroll
    for (int bd = 0; bd < D / 32; ++bd)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        acc[bd][r] *= alpha;
  }

  // O^T += V^T . P^T for the values in V slot SLOT.
  template <int SLOT>
  __device__ __forceinline__ static void pv(const Bases &bs, const h8 (&pf)[BN / 16],
                                            f16v (&acc)[D / 32]) {
    constexpr int VGRP = D / 32 < 4 ? D / 32 : 4; // dim blocks read together
#pragma unroll
    for (int b0 = 0; b0 < D / 32; b0 += VGRP) {
      h8 vf[VGRP][BN / 16];
#pragma unroll
      for (int bd = 0; bd < VGRP; ++bd)
#pragma unroll
        for (int c = 0; c < BN / 16; ++c)
          vf[bd][c] = read_v<SLOT>(bs, b0 + bd, c);
#pragma unroll
      for (int bd = 0; bd < VGRP; ++bd)
#pragma unroll
        for (int c = 0; c < BN / 16; ++c)
          acc[b0 + bd] = mfma(vf[bd][c], pf[c], acc[b0 + bd]);
    }
  }

  // The kernel's view of this element type.
  struct QF {
    h8 v[D / 16];
  };
  typedef h8 PF[BN / 16];
  // Q rows as MFMA B operands: dims 16 c + 8 g .. +7 of row m.
  __device__ __forceinline__ static void load_q(const uint8_t *Qh, int64_t m, int64_t sm,
                                                QF &qf) {
    const int g = (threadIdx.x & 63) >> 5;
#pragma unroll
    for (int c = 0; c < D / 16; ++c)
      qf.v[c] = 16 * c + 8 * g < DR
                    ? *reinterpret_cast<const h8 *>(Qh + (m * sm + 16 * c + 8 * g) * 2)
                    : h8{};
  }
  __device__ __forceinline__ static uint32_t k_bytes(int64_t n_ctx, int64_t sm) {
    return (uint32_t)(((n_ctx - 1) * sm + DR) * 2);
  }
  __device__ __forceinline__ static uint32_t v_bytes(int64_t n_ctx, int64_t sm) {
    return k_bytes(n_ctx, sm);
  }
  __device__ __forceinline__ static void kv_offsets(int wave, int64_t k_sm, int64_t v_sm,
                                                    uint32_t (&ko)[DMA], uint32_t (&vo)[DMA]) {
    dma_offsets<false>(wave, k_sm, ko);
    dma_offsets<true>(wave, v_sm, vo);
  }
  __device__ __forceinline__ static void issue_k(const i32x4_t &rsrc, const uint32_t (&off)[DMA],
                                                 int64_t sm, int j, uint32_t lds, int wave) {
    issue(rsrc, off, sm, j, lds, wave);
  }
  __device__ __forceinline__ static void issue_v(const i32x4_t &rsrc, const uint32_t (&off)[DMA],
                                                 int64_t sm, int j, uint32_t lds, int wave) {
    issue(rsrc, off, sm, j, lds, wave);
  }
  template <int SLOT>
  __device__ __forceinline__ static void qk(const Bases &bs, const QF &qf, f16v (&s)[BN / 32]) {
    qk<SLOT>(bs, qf.v, s);
  }
  // O = acc / l_i.  Lane l holds, per dim block bd and register quad q, dims
  // 32 bd + 8 q + 4 g .. +3 of row m.
  __device__ __forceinline__ static void store_o(const f16v (&acc)[D / 32], float l_i,
                                                 uint8_t *Orow) {
    const int g = (threadIdx.x & 63) >> 5;
#pragma unroll
    for (int bd = 0; bd < D / 32; ++bd)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (32 * bd + 8 * q >= DR) // the layout's dims past the real head dim
          continue;
        h4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          o[e] = (elt)(acc[bd][4 * q + e] / l_i);
        *reinterpret_cast<h4 *>(Orow + (32 * bd + 8 * q + 4 * g) * 2) = o;
      }
  }
};

// The K/V loop is software-pipelined: iteration j holds S_j in registers,
// computes S_{j+1} (MFMA) while it turns S_j into P_j (VALU), then adds
// P_j V_j.  K and V have two LDS slots each, K one block ahead of V:
// iteration j first issues the loads of K_{j+2} (into K_j's slot) and
// V_{j+1} (into V_{j-1}'s slot), and its closing barrier makes them visible.
// Block j uses K slot j%2 and V slot j%2, a template constant: each segment
// runs in pairs of iterations, with a single one first when it starts at an
// odd block and last when it ends at one.
// A: the element type's fragments (AttnFwd<HD, BF> here, AttnFwd8<HD> for
// e5m2).
template <bool CAUSAL, class A> __device__ __forceinline__ void attn_fwd_body(const AttnArgs &p) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[4 * A::TILE];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 5;
  // Program order: the 8 XCDs take contiguous runs of programs (a head's
  // K/V stays in one L2), and within a head the longest causal rows first.
  const int nm = p.N_CTX / A::BM, nwg = gridDim.x, b = blockIdx.x;
  const int t = (nwg % 8 == 0) ? (b % 8) * (nwg / 8) + b / 8 : b;
  const int hz = t / nm, start_m = CAUSAL ? nm - 1 - t % nm : t % nm;
  const int z = hz / p.H, h = hz % p.H;
  const uint8_t *Qh = static_cast<const uint8_t *>(p.Q) + (z * p.q_sz + h * p.q_sh) * A::ESZ;
  const uint8_t *Kh = static_cast<const uint8_t *>(p.K) + (z * p.k_sz + h * p.k_sh) * A::ESZ;
  const uint8_t *Vh = static_cast<const uint8_t *>(p.V) + (z * p.v_sz + h * p.v_sh) * A::ESZ;
  const int m = start_m * A::BM + 32 * wave + (lane & 31);

  typename A::QF qf;
  A::load_q(Qh, m, p.q_sm, qf);

  const i32x4_t rk = make_rsrc(Kh, A::k_bytes(p.N_CTX, p.k_sm));
  const i32x4_t rv = make_rsrc(Vh, A::v_bytes(p.N_CTX, p.v_sm));
  uint32_t ko[A::DMA], vo[A::DMA];
  A::kv_offsets(wave, p.k_sm, p.v_sm, ko, vo);
  const uint32_t k_lds = lds_addr(smem), v_lds = k_lds + 2 * A::TILE;
  typename A::Bases bs;
  A::bases(k_lds, v_lds, bs);

  // LoopSplit form of the K/V loop (keys [0, N_CTX), predicate start_n >=
  // causal_start): unmasked blocks [0, n_main), masked [n_main, n_end).
  // N_CTX and causal_start are multiples of BM, itself a multiple of BN.
  const int causal_start = CAUSAL ? start_m * A::BM : p.N_CTX;
  const int n_main = causal_start / A::BN;
  const int n_end = CAUSAL ? (causal_start + A::BM) / A::BN : n_main;

  float m_i = -INFINITY, l_i = 1.0f;
  typename A::f16v acc[A::D / 32], s[A::BN / 32];
#pragma unroll
  for (int bd = 0; bd < A::D / 32; ++bd)
    acc[bd] = typename A::f16v{};

  A::issue_k(rk, ko, p.k_sm, 0, k_lds, wave);
  A::issue_v(rv, vo, p.v_sm, 0, v_lds, wave);
  if (n_end > 1)
    A::issue_k(rk, ko, p.k_sm, 1, k_lds + A::TILE, wave);
  __builtin_amdgcn_s_waitcnt(0x7 << 4); // vmcnt(0)
  __syncthreads();
  A::template qk<0>(bs, qf, s);
  __syncthreads(); // K slot 0 is refilled by iteration 0

  auto iter = [&](int j, auto mask, auto slot) {
    constexpr bool MASK = decltype(mask)::value;
    constexpr int SL = decltype(slot)::value;
    if (j + 2 < n_end)
      A::issue_k(rk, ko, p.k_sm, j + 2, k_lds + SL * A::TILE, wave);
    if (j + 1 < n_end)
      A::issue_v(rv, vo, p.v_sm, j + 1, v_lds + (1 - SL) * A::TILE, wave);
    typename A::f16v sn[A::BN / 32];
    A::template qk<1 - SL>(bs, qf, sn); // S_{j+1} (a stale slot after the last block: unused)
    // On-band blocks whose keys all lie past this wave's 32 rows add exactly
    // nothing (p = 0, alpha = 1, as for the blocks past the diagonal): the
    // wave skips their softmax and P V.
    const bool live = !MASK || j * A::BN <= start_m * A::BM + 32 * wave + 31;
    if (live) {
      typename A::PF pf;
      A::template softmax<MASK>(s, j * A::BN, m, p.qk_scale, acc, m_i, l_i, pf);
      A::template pv<SL>(bs, pf, acc);
    }
#pragma unroll
    for (int b2 = 0; b2 < A::BN / 32; ++b2)
      s[b2] = sn[b2];
    __builtin_amdgcn_s_waitcnt(0x7 << 4); // vmcnt(0): this wave's loads of K_{j+2}, V_{j+1}
    __syncthreads();
  };
  auto segment = [&](int j, int j_end, auto mask) {
    if (j < j_end && (j & 1)) {
      iter(j, mask, std::integral_constant<int, 1>());
      ++j;
    }
    for (; j + 1 < j_end; j += 2) {
      iter(j, mask, std::integral_constant<int, 0>());
      iter(j + 1, mask, std::integral_constant<int, 1>());
    }
    if (j < j_end)
      iter(j, mask, std::integral_constant<int, 0>());
  };
  segment(0, n_main, std::false_type());
  segment(n_main, n_end, std::true_type());

  // Epilogue: M = m_i + log2(l_i); O = acc / l_i.
  A::store_o(acc, l_i,
             static_cast<uint8_t *>(p.O) +
                 (z * p.o_sz + h * p.o_sh + (int64_t)m * p.o_sm) * A::ESZ);
  if (g == 0)
    p.M[(int64_t)hz * p.N_CTX + m] = m_i + __builtin_log2f(l_i);
}

template <bool CAUSAL, int HD, bool BF, int BM = 128, int BN = 64>
__global__ void __launch_bounds__(BM * 2, HD >= 256 ? 1 : 2) attn_fwd_kernel(AttnArgs p) {
  attn_fwd_body<CAUSAL, AttnFwd<HD, BF, BM, BN>>(p);
}

} // namespace txk
