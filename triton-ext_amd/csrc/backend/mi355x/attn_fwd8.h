// Fused attention forward for gfx950, fp8 e5m2: the tutorial's fp8 provider
// (R:pass/LoopSplit/06-fused-attention.py:774-779: q, k, v cast to
// float8_e5m2, v stored key-contiguous; :81-82 p.to(tl.float8e5) before
// p @ v; :238 o in q's type), HEAD_DIM 16, 32, 64, 128 or 256, fp32
// statistics and accumulator.  HEAD_DIM 16 and 32 run in the layout of 64
// (one S^T MFMA takes 64 dims): K's chunks and V^T's dim rows past the real
// head dim load as zeros (out-of-range buffer offsets), Q's bytes past it are
// zero and O's are not stored.  The pipeline, split and program order are attn_fwd_body's
// (attn_fwd.h); this file holds the element type's fragments.
//
// Per K/V block of BN = 64 (or 32) keys and wave of 32 query rows (BM / 32
// waves):
//   S^T = K . Q^T    v_mfma_f32_32x32x64_f8f6f4 (e5m2 x e5m2), one per 32
//                    keys and 64 dims.  Lane l feeds A row l%32 with key
//                    pi(l%32), pi(8i + 4g + j) = 16g + 4i + j, so the S^T
//                    registers r of lane l hold keys 16 (l/32) + r of each
//                    32-key block: 16 consecutive keys per lane;
//   P                p converted to e5m2 with v_cvt_pk_bf8_f32 (round to
//                    nearest even), packed in key order: byte 16 b + r of
//                    lane l is key 32 b + 16 (l/32) + r;
//   O^T += V^T . P^T one MFMA per 32 dims: A := V^T rows (dims), whose keys
//                    are contiguous in memory and in LDS, read as the same
//                    two 16-key chunks (l/32 and 2 + l/32) that P holds.
//                    With BN = 32 the block has only chunk l/32: the other
//                    half of both operands is zero bytes in registers, so
//                    the MFMA adds exactly the block's 32 products.
// The two dots use any K order that is the same for both operands; the
// order above needs no transposes and no lane exchanges.
//
// LDS (16-byte chunk c of row r stored at c ^ swizzle(r)):
//   K rows (keys) of HEAD_DIM bytes: 64-byte rows ((r >> 2) & 1) |
//     ((r >> 3) & 2); 128-byte rows ((r >> 1) & 3) | ((r >> 2) & 4);
//     256-byte rows (r & 7) | ((r >> 1) & 8).  The 16 keys pi(0..15) (or
//     pi(16..31)) that one ds_read_b128 pass reads land in 16 different
//     16-byte bank groups;
//   V^T rows (dims) of BN bytes (the block's keys): (r >> 2) & 3 for 64-byte
//     rows, (r >> 3) & 1 for 32-byte rows, likewise for dims 0..15 of a pass.
#pragma once

#include "attn_fwd.h"

namespace txk {

// BM_ x BN_: BLOCK_M 64 or 128 (one wave per 32 query rows) by BLOCK_N 64 or
// 32.  The P V MFMA takes 64 keys at once; a block of 32 fills half of it.
template <int HD, int BM_ = 128, int BN_ = 64> struct AttnFwd8 {
  // D: the head dim of the layout (64 for HEAD_DIM 16 and 32); DR: the real one
  static constexpr int BM = BM_, BN = BN_, D = HD < 64 ? 64 : HD, DR = HD, NW = BM_ / 32,
                       ESZ = 1;
  static constexpr int TILE = BN * D;          // K: BN x D bytes; V^T: D x BN bytes
  // LW: the waves that stage a K/V block, all of them unless the block holds
  // fewer 1 KiB loads than there are waves (2 KiB for 4 waves at head dims
  // 16 and 32 with 128 x 32 blocks: waves 0 and 1 load, 2 and 3 only wait
  // at the barriers that publish every block).
  static constexpr int LW = TILE / 1024 < NW ? TILE / 1024 : NW;
  static constexpr int DMA = TILE / 1024 / LW; // 16-byte loads per lane per tile: 1 .. 8
  static constexpr int KCPR = D / 16;          // K: 16-byte chunks per row
  static constexpr int VCPR = BN / 16;         // V^T: 16-byte chunks per dim row
  static constexpr uint32_t kOOB = 0x80000000u;
  static_assert(D == 64 || D == 128 || D == 256, "head dims 16 .. 256");
  static_assert(DR == D || (D == 64 && (DR == 16 || DR == 32)), "16 and 32 in the layout of 64");
  static_assert((BM == 64 || BM == 128) && (BN == 32 || BN == 64), "the tutorial's blocks");
  static_assert(LW >= 1 && DMA >= 1 && DMA * LW * 1024 == TILE, "whole 1 KiB loads per wave");
  typedef float f16v __attribute__((ext_vector_type(16)));

  __device__ __forceinline__ static f16v mfma(const i32x8_t &a, const i32x8_t &b,
                                              const f16v &c) {
    // formats 1, 1: e5m2 x e5m2; zero scale operands: the unscaled MFMA.
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 1, 1, 0, 0, 0, 0);
  }
  __device__ __forceinline__ static int kswz(int r) {
    return D == 64    ? ((r >> 2) & 1) | ((r >> 3) & 2)
           : D == 128 ? ((r >> 1) & 3) | ((r >> 2) & 4)
                      : (r & 7) | ((r >> 1) & 8);
  }
  __device__ __forceinline__ static int vswz(int r) {
    return BN == 64 ? (r >> 2) & 3 : (r >> 3) & 1;
  }
  // key of A row R of the S^T MFMA
  __device__ __forceinline__ static int pi(int R) {
    return 16 * ((R >> 2) & 1) + 4 * (R >> 3) + (R & 3);
  }

  // Q rows as MFMA B operands: bytes 64 c + 32 (l/32) .. +31 of row m.
  struct QF {
    i32x8_t v[D / 64];
  };
  typedef i32x8_t PF;

  __device__ __forceinline__ static void load_q(const uint8_t *Qh, int64_t m, int64_t sm,
                                                QF &qf) {
    const int g = (threadIdx.x & 63) >> 5;
#pragma unroll
    for (int c = 0; c < D / 64; ++c) {
      const int b0 = 64 * c + 32 * g; // the lane's first byte of the row
      const i32x4_t *src = reinterpret_cast<const i32x4_t *>(Qh + m * sm + b0);
      const i32x4_t lo = b0 < DR ? src[0] : i32x4_t{0, 0, 0, 0};
      const i32x4_t hi = b0 + 16 < DR ? src[1] : i32x4_t{0, 0, 0, 0};
      qf.v[c] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    }
  }
  __device__ __forceinline__ static uint32_t k_bytes(int64_t n_ctx, int64_t sm) {
    return (uint32_t)((n_ctx - 1) * sm + DR);
  }
  // v is [HEAD_DIM][N_CTX] per head (key-contiguous), sm the dim stride.
  __device__ __forceinline__ static uint32_t v_bytes(int64_t n_ctx, int64_t sm) {
    return (uint32_t)((DR - 1) * sm + n_ctx);
  }

  __device__ __forceinline__ static void dma16(uint32_t voff, const i32x4_t &rsrc, uint32_t soff,
                                               uint32_t lds) {
    asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(rsrc), "s"(soff),
                 "{m0}"(lds)
                 : "memory");
  }
  // Per-lane source offsets of the wave's DMA loads: load u of wave w fills
  // 1 KiB of LDS.  K: rows 1024/D (DMA w + u) + i/KCPR of D bytes; V^T: dim
  // rows 1024/BN (DMA w + u) + i/VCPR of BN bytes.  Lane i's chunk position holds the
  // source chunk (position ^ swizzle(row)).  K chunks and V^T dim rows past
  // the real head dim take kOOB (zeros).
  __device__ __forceinline__ static void kv_offsets(int wave, int64_t k_sm, int64_t v_sm,
                                                    uint32_t (&ko)[DMA], uint32_t (&vo)[DMA]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int u = 0; u < DMA; ++u) {
      const int kr = (1024 / D) * (DMA * wave + u) + lane / KCPR, kp = lane % KCPR;
      const int kc = kp ^ kswz(kr);
      ko[u] = 16 * kc >= DR ? kOOB : (uint32_t)(kr * k_sm + 16 * kc);
      const int vr = (1024 / BN) * (DMA * wave + u) + lane / VCPR, vp = lane % VCPR;
      vo[u] = vr >= DR ? kOOB : (uint32_t)(vr * v_sm + 16 * (vp ^ vswz(vr)));
    }
  }
  // K block j: rows j BN .. of the key-major K; V block j: bytes j BN .. of
  // every dim row.
  // Neither issues from waves past LW (`wave` is wave-uniform).
  __device__ __forceinline__ static void issue_k(const i32x4_t &rsrc, const uint32_t (&off)[DMA],
                                                 int64_t sm, int j, uint32_t lds, int wave) {
    if (LW < NW && wave >= LW)
      return;
#pragma unroll
    for (int u = 0; u < DMA; ++u)
      dma16(off[u], rsrc, (uint32_t)((int64_t)j * BN * sm), lds + (DMA * wave + u) * 1024);
  }
  __device__ __forceinline__ static void issue_v(const i32x4_t &rsrc, const uint32_t (&off)[DMA],
                                                 int64_t, int j, uint32_t lds, int wave) {
    if (LW < NW && wave >= LW)
      return;
#pragma unroll
    for (int u = 0; u < DMA; ++u)
      dma16(off[u], rsrc, (uint32_t)(j * BN), lds + (DMA * wave + u) * 1024);
  }

  // Per-lane LDS addresses (slot 0) of the fragment reads; the key block b
  // and dim block bd enter as immediate offsets (the swizzles do not depend
  // on key bit 5 or dim bit 5):
  //   K, dim chunk pair c, half e: key pi(l%32), chunk 4c + 2(l/32) + e;
  //   V^T, half e: dim l%32, chunk l/32 + 2e.
  struct Bases {
    uint32_t k[D / 64][2], v[BN / 32];
  };
  __device__ __forceinline__ static void bases(uint32_t k_lds, uint32_t v_lds, Bases &bs) {
    const int lane = threadIdx.x & 63, g = lane >> 5, r = lane & 31;
    const int key = pi(r);
#pragma unroll
    for (int c = 0; c < D / 64; ++c)
#pragma unroll
      for (int e = 0; e < 2; ++e)
        bs.k[c][e] = k_lds + key * D + 16 * ((4 * c + 2 * g + e) ^ kswz(key));
#pragma unroll
    for (int e = 0; e < BN / 32; ++e)
      bs.v[e] = v_lds + r * BN + 16 * ((g + 2 * e) ^ vswz(r));
  }

  __device__ __forceinline__ static i32x4_t lds16(uint32_t a) {
    typedef __attribute__((address_space(3))) i32x4_t lds_i32x4;
    return *(const lds_i32x4 *)(uintptr_t)a;
  }
  template <int SLOT>
  __device__ __forceinline__ static i32x8_t read_k(const Bases &bs, int b, int c) {
    const uint32_t o = SLOT * TILE + b * 32 * D;
    const i32x4_t lo = lds16(bs.k[c][0] + o), hi = lds16(bs.k[c][1] + o);
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  }
  template <int SLOT>
  __device__ __forceinline__ static i32x8_t read_v(const Bases &bs, int bd) {
    const uint32_t o = SLOT * TILE + bd * 32 * BN;
    const i32x4_t lo = lds16(bs.v[0] + o);
    const i32x4_t hi = BN == 64 ? lds16(bs.v[BN / 32 - 1] + o) : i32x4_t{0, 0, 0, 0};
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  }

  __device__ __forceinline__ static float xmax(float v) { return AttnFwd<HD, false>::xmax(v); }
  __device__ __forceinline__ static float xsum(float v) { return AttnFwd<HD, false>::xsum(v); }

  // S^T block of the keys in K slot SLOT: lane holds query row l%32.
  template <int SLOT>
  __device__ __forceinline__ static void qk(const Bases &bs, const QF &qf, f16v (&s)[BN / 32]) {
    i32x8_t kf[BN / 32][D / 64];
#pragma unroll
    for (int b = 0; b < BN / 32; ++b)
#pragma unroll
      for (int c = 0; c < D / 64; ++c)
        kf[b][c] = read_k<SLOT>(bs, b, c);
#pragma unroll
    for (int b = 0; b < BN / 32; ++b) {
      s[b] = f16v{};
#pragma unroll
      for (int c = 0; c < D / 64; ++c)
        s[b] = mfma(kf[b][c], qf.v[c], s[b]);
    }
  }

  // Softmax of one block (the tutorial's arithmetic) for the lane's query
  // row m, keys n0 + 32 b + 16 g + r: updates m_i and l_i, rescales acc by
  // alpha and returns P as e5m2 bytes in key order.  MASK: on-band form.
  template <bool MASK>
  __device__ __forceinline__ static void softmax(f16v (&s)[BN / 32], int n0, int m,
                                                 float qk_scale, f16v (&acc)[D / 32],
                                                 float &m_i, float &l_i, PF &pf) {
    const int g = (threadIdx.x & 63) >> 5;
    float m_ij;
    if constexpr (MASK) {
      float mx = -INFINITY;
#pragma unroll
      for (int b = 0; b < BN / 32; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
#pragma clang fp contract(off)
          const int n = n0 + 32 * b + 16 * g + r;
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
    for (int w = 0; w < 8; ++w) {
      const int b = w / 4, r = 4 * (w % 4);
      if (b >= BN / 32) { // the MFMA's keys past a block of 32
        pf[w] = 0;
        continue;
      }
      const int lo = __builtin_amdgcn_cvt_pk_bf8_f32(s[b][r], s[b][r + 1], 0, false);
      pf[w] = __builtin_amdgcn_cvt_pk_bf8_f32(s[b][r + 2], s[b][r + 3], lo, true);
    }
#pragma unroll
    for (int bd = 0; bd < D / 32; ++bd)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        acc[bd][r] *= alpha;
  }

  // O^T += V^T . P^T for the values in V slot SLOT.
  template <int SLOT>
  __device__ __forceinline__ static void pv(const Bases &bs, const PF &pf,
                                            f16v (&acc)[D / 32]) {
    i32x8_t vf[D / 32];
#pragma unroll
    for (int bd = 0; bd < D / 32; ++bd)
      vf[bd] = read_v<SLOT>(bs, bd);
#pragma unroll
    for (int bd = 0; bd < D / 32; ++bd)
      acc[bd] = mfma(vf[bd], pf, acc[bd]);
  }

  // O = e5m2(acc / l_i), round to nearest even.  Lane l holds, per dim block
  // bd and register quad q, dims 32 bd + 8 q + 4 (l/32) .. +3 of row m: one
  // 4-byte store each.
  __device__ __forceinline__ static void store_o(const f16v (&acc)[D / 32], float l_i,
                                                 uint8_t *Orow) {
    const int g = (threadIdx.x & 63) >> 5;
#pragma unroll
    for (int bd = 0; bd < D / 32; ++bd)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (32 * bd + 8 * q >= DR) // the layout's dims past the real head dim
          continue;
        int w = __builtin_amdgcn_cvt_pk_bf8_f32(acc[bd][4 * q] / l_i, acc[bd][4 * q + 1] / l_i,
                                                0, false);
        w = __builtin_amdgcn_cvt_pk_bf8_f32(acc[bd][4 * q + 2] / l_i, acc[bd][4 * q + 3] / l_i, w,
                                            true);
        *reinterpret_cast<int *>(Orow + 32 * bd + 8 * q + 4 * g) = w;
      }
  }
};

template <bool CAUSAL, int HD, int BM = 128, int BN = 64>
__global__ void __launch_bounds__(BM * 2, HD >= 256 ? 1 : 2) attn_fwd8_kernel(AttnArgs p) {
  attn_fwd_body<CAUSAL, AttnFwd8<HD, BM, BN>>(p);
}

} // namespace txk
