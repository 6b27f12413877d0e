// LDS-staged MFMA tile kernel for gfx950: C[M,N] = epilogue(A[M,K] . B[K,N]),
// A, B and C row-major.
//
// One workgroup computes a BM x BN tile of C; its WM x WN waves each own a
// (BM/WM) x (BN/WN) sub-tile made of 32x32 MFMA blocks whose accumulators stay
// in registers (VGPR/AGPR) for the whole K loop.
//
// Operand staging (per K step of BK elements):
//   A: 16-byte global loads, consecutive threads along a row (coalesced), into
//      an LDS tile of BM rows x BK elements, K-contiguous.
//   B: arrives N-contiguous, but an MFMA lane needs K-contiguous data for one
//      column.  Each thread loads an E x E block (E = 16 bytes / element:
//      8x8 bf16/fp16, 16x16 int8/fp8) as E row loads of 16 bytes, transposes
//      it in registers with byte permutes, and stores E K-contiguous rows, so
//      the LDS B tile is BN rows x BK elements like A's.
//   Rows are XOR-swizzled in 16-byte chunks (txk::lds_off) and the LDS tile
//   is double-buffered: the global loads for step k+1 are in flight while
//   step k's MFMAs run, with one barrier per step.
//
// K loop (the LoopSplit form, planned on the host): k_main_steps full steps
// with unmasked loads, then k_masked_steps steps (one with the split, all of
// them with TX_FLAG_NO_LOOP_SPLIT) whose loads zero-fill k >= K, the
// tl.load(mask, other=0) semantics.  Only the MFMA sub-steps that the last
// step's k_tail covers are issued.  Tiles crossing M or N take the masked
// instantiation; interior tiles never test a bound.
#pragma once

#include <type_traits>

#include "tile_common.h"

namespace txk {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
typedef __attribute__((__vector_size__(16 * sizeof(int)))) int i32x16_t;
typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4_t;
typedef __attribute__((__vector_size__(8 * sizeof(int)))) int i32x8_t;

enum OpKind { OP_BF16 = 0, OP_F16 = 1, OP_I8 = 2, OP_F8 = 3 };
enum EpiKind {
  EPI_F32 = 0,           // store the fp32 accumulator
  EPI_BF16 = 1,          // RNE to bf16
  EPI_F16 = 2,           // RNE to fp16
  EPI_I32 = 3,           // store the int32 accumulator
  EPI_ROWCOL_BF16 = 4,   // bf16((float(acc) * sa[m]) * sb[n])
  EPI_BLOCK128_BF16 = 5, // per-128-K-block scaled fp32 acc, RNE to bf16
  EPI_BLOCK128_F32 = 6,  // per-128-K-block scaled fp32 acc
  EPI_MX_F32 = 7,        // e8m0 per-32-K scales applied by the MFMA, fp32 C
  EPI_MX_BF16 = 8,       // the same, RNE to bf16
};

template <int OP> struct OpTraits;
// ELT: bytes per element; KM: K per MFMA; CPL: 16-byte chunks per lane per
// MFMA operand.
template <> struct OpTraits<OP_BF16> {
  static constexpr int ELT = 2, KM = 16, CPL = 1;
  typedef f32x16_t Acc;
};
template <> struct OpTraits<OP_F16> {
  static constexpr int ELT = 2, KM = 16, CPL = 1;
  typedef f32x16_t Acc;
};
template <> struct OpTraits<OP_I8> {
  static constexpr int ELT = 1, KM = 32, CPL = 1;
  typedef i32x16_t Acc;
};
template <> struct OpTraits<OP_F8> {
  static constexpr int ELT = 1, KM = 64, CPL = 2;
  typedef f32x16_t Acc;
};

template <int CPL> struct Frag {
  u32x4 v[CPL];
};

// One 32x32 MFMA block: acc += a . b over KM elements of K.
__device__ __forceinline__ f32x16_t mfma(OpTraits<OP_BF16>, const Frag<1> &a,
                                         const Frag<1> &b, f32x16_t acc) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(
      __builtin_bit_cast(bf16x8_t, a.v[0]), __builtin_bit_cast(bf16x8_t, b.v[0]),
      acc, 0, 0, 0);
}
__device__ __forceinline__ f32x16_t mfma(OpTraits<OP_F16>, const Frag<1> &a,
                                         const Frag<1> &b, f32x16_t acc) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(
      __builtin_bit_cast(f16x8_t, a.v[0]), __builtin_bit_cast(f16x8_t, b.v[0]),
      acc, 0, 0, 0);
}
__device__ __forceinline__ i32x16_t mfma(OpTraits<OP_I8>, const Frag<1> &a,
                                         const Frag<1> &b, i32x16_t acc) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(
      __builtin_bit_cast(i32x4_t, a.v[0]), __builtin_bit_cast(i32x4_t, b.v[0]),
      acc, 0, 0, 0);
}
__device__ __forceinline__ f32x16_t mfma(OpTraits<OP_F8>, const Frag<2> &a,
                                         const Frag<2> &b, f32x16_t acc) {
  i32x8_t av, bv;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    av[i] = (int)a.v[0][i];
    av[4 + i] = (int)a.v[1][i];
    bv[i] = (int)b.v[0][i];
    bv[4 + i] = (int)b.v[1][i];
  }
  // format 0 for both operands = fp8 e4m3; scale operands 0 = no scaling.
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, acc, 0, 0, 0,
                                                         0, 0, 0);
}

struct GemmArgs {
  const uint8_t *A;
  const uint8_t *B;
  void *C;
  const float *sa; // ROWCOL: [M]; BLOCK128: [M][sa_ld]; MX: uint8 [M][sa_ld]
  const float *sb; // ROWCOL: [N]; BLOCK128: [ceil(K/128)][sb_ld]; MX: uint8 [N][sa_ld]
  int64_t M, N, K;
  int64_t lda, ldb, ldc; // row strides in elements
  int32_t tiles_m, tiles_n;
  int32_t k_main_steps;   // unmasked K steps
  int32_t k_masked_steps; // masked K steps after them
  int32_t last_ks;        // MFMA sub-steps issued in the final K step
  int32_t group_m;        // tile rows per group in the tile order
  int32_t sa_ld, sb_ld; // MX: sa_ld = bytes per scale row = K / 32 groups
  int32_t accumulate;   // fp32 / int32 C: C = C + A . B (tl.dot's acc operand)
  // Split-K (the 256x256 tiles): split_k > 1 launches split_k workgroups per
  // tile (blockIdx.y); range z runs K steps [z split_steps, (z + 1)
  // split_steps) of its tile, the last range the rest, which the K-loop
  // fields above describe, and stores its 32-bit sums at C + z M ldc.
  int32_t split_k = 1;
  int32_t split_steps = 0;
};

// The arguments of this workgroup's K range under split-K: A, B and the
// 128-block scales advanced to the range's first K step, C to its partial,
// and K with the loop fields of a range of whole steps (every range but the
// last).  BK: K elements a step (bytes for 8-bit); FULL_KS: MFMA sub-steps
// of a whole step; ELT: bytes an element; BT: B K-major; BLOCK: 128-block
// scales (BK is then 128: a step is one scale block).
template <int BK, int FULL_KS, int ELT, bool BT, bool BLOCK>
__device__ __forceinline__ GemmArgs split_k_args(const GemmArgs &p) {
  GemmArgs q = p;
  if (p.split_k <= 1)
    return q;
  const int z = blockIdx.y;
  const int64_t k0 = (int64_t)z * p.split_steps * BK;
  q.A = p.A + k0 * ELT;
  q.B = p.B + (BT ? k0 * ELT : k0 * p.ldb * ELT);
  q.C = static_cast<uint8_t *>(p.C) + (int64_t)z * p.M * p.ldc * 4;
  if (BLOCK) {
    q.sa = p.sa + k0 / 128;
    q.sb = p.sb + (k0 / 128) * p.sb_ld;
  }
  q.K = p.K - k0;
  if (z < p.split_k - 1) {
    q.K = (int64_t)p.split_steps * BK;
    q.k_main_steps = p.split_steps;
    q.k_masked_steps = 0;
    q.last_ks = FULL_KS;
  }
  return q;
}

// Workgroups are dispatched round-robin over the 8 XCDs (each with its own
// L2), so workgroup b runs on XCD b % 8.  Renumber so that each XCD gets a
// contiguous run of tile ids, then walk tiles in groups of group_m tile rows
// (column-major inside a group): an XCD's tiles then share A rows and B
// columns in its L2.
__device__ __forceinline__ void tile_coords(const GemmArgs &p, int &tm,
                                            int &tn) {
  const int nwg = gridDim.x, b = blockIdx.x;
  int t = (nwg % 8 == 0) ? (b % 8) * (nwg / 8) + b / 8 : b;
  const int width = p.group_m * p.tiles_n;
  const int group = t / width;
  const int first_m = group * p.group_m;
  int gsz = p.tiles_m - first_m;
  gsz = gsz < p.group_m ? gsz : p.group_m;
  const int r = t - group * width;
  tm = first_m + r % gsz;
  tn = r / gsz;
}

template <int OP, int BM, int BN, int BK, int WM, int WN, int EPI>
struct GemmTile {
  typedef OpTraits<OP> T;
  typedef typename T::Acc Acc;
  static constexpr int ELT = T::ELT, KM = T::KM, CPL = T::CPL;
  static constexpr int NT = WM * WN * 64;
  static constexpr int RB = BK * ELT;  // bytes per LDS row
  static constexpr int NCH = RB / 16;  // 16-byte chunks per row
  static constexpr int E = 16 / ELT;   // elements per chunk
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int FM = WTM / 32, FN = WTN / 32;
  static constexpr int KS = BK / KM;   // MFMA sub-steps per K step
  static constexpr int A_LOADS = BM * NCH / NT;
  static constexpr int B_BLOCKS = (BK / E) * (BN / E);
  static constexpr int B_PER = (B_BLOCKS + NT - 1) / NT;
  static constexpr bool SCALED = EPI == EPI_BLOCK128_BF16 || EPI == EPI_BLOCK128_F32;
  static constexpr int A_BYTES = BM * RB, B_BYTES = BN * RB;
  static constexpr int LDS_BYTES = 2 * (A_BYTES + B_BYTES) + (SCALED ? 2 * BM * 4 : 0);

  static_assert(RB % 16 == 0 && (NCH & (NCH - 1)) == 0, "row must be 2^n chunks");
  static_assert(BK % KM == 0, "BK must be a multiple of the MFMA K");
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be 32x32 blocks");
  static_assert((BM * NCH) % NT == 0, "A tile must split evenly over threads");
  static_assert(!SCALED || BK == 128, "block scales need BK == 128");
  static_assert(!SCALED || BM <= NT, "scale staging: one row per thread");

  template <bool MASK_MN>
  __device__ __forceinline__ static void run(const GemmArgs &p, uint8_t *smem,
                                             int64_t m0, int64_t n0) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    uint8_t *As = smem;
    uint8_t *Bs = smem + 2 * A_BYTES;
    float *Ss = reinterpret_cast<float *>(smem + 2 * (A_BYTES + B_BYTES));

    Acc acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          acc[i][j][r] = 0;

    u32x4 ra[A_LOADS];
    u32x4 rb[B_PER][E];
    float rs = 0.f; // this thread's row scale for the staged K step
    const u32x4 zero = {0u, 0u, 0u, 0u};

    auto load = [&](int kt, auto mask_k_tag) {
      constexpr bool MASK_K = decltype(mask_k_tag)::value;
      const int64_t k0 = (int64_t)kt * BK;
#pragma unroll
      for (int i = 0; i < A_LOADS; ++i) {
        const int id = tid + i * NT, row = id / NCH, ch = id % NCH;
        const int64_t gm = m0 + row, gk = k0 + (int64_t)ch * E;
        const bool ok = (!MASK_MN || gm < p.M) && (!MASK_K || gk < p.K);
        ra[i] = ok ? *reinterpret_cast<const u32x4 *>(p.A + (gm * p.lda + gk) * ELT)
                   : zero;
        if (MASK_K && gk + E > p.K) {
          // the chunk crosses K (K need not fill whole chunks): keep the
          // bytes of elements below K (B's rows past K are zero-filled)
          const int64_t vb = (p.K - gk) * ELT;
#pragma unroll
          for (int w = 0; w < 4; ++w)
            ra[i][w] &= vb >= 4 * w + 4 ? 0xffffffffu
                        : vb <= 4 * w   ? 0u
                                        : (1u << (8 * (vb - 4 * w))) - 1u;
        }
      }
#pragma unroll
      for (int i = 0; i < B_PER; ++i) {
        const int b = tid + i * NT;
        if (B_BLOCKS % NT == 0 || b < B_BLOCKS) {
          const int nb = b % (BN / E), kb = b / (BN / E);
          const int64_t gn = n0 + (int64_t)nb * E;
#pragma unroll
          for (int j = 0; j < E; ++j) {
            const int64_t gk = k0 + (int64_t)kb * E + j;
            const bool ok = (!MASK_MN || gn < p.N) && (!MASK_K || gk < p.K);
            rb[i][j] = ok ? *reinterpret_cast<const u32x4 *>(p.B + (gk * p.ldb + gn) * ELT)
                          : zero;
          }
        }
      }
      if (SCALED && tid < BM) {
        const int64_t gm = m0 + tid;
        rs = (!MASK_MN || gm < p.M) ? p.sa[gm * p.sa_ld + kt] : 0.f;
      }
    };
    using Unmasked = std::integral_constant<bool, false>;
    using Masked = std::integral_constant<bool, true>;

    auto store = [&](int buf) {
      uint8_t *as = As + buf * A_BYTES;
      uint8_t *bs = Bs + buf * B_BYTES;
#pragma unroll
      for (int i = 0; i < A_LOADS; ++i) {
        const int id = tid + i * NT, row = id / NCH, ch = id % NCH;
        *reinterpret_cast<u32x4 *>(as + lds_off(row, ch, NCH)) = ra[i];
      }
#pragma unroll
      for (int i = 0; i < B_PER; ++i) {
        const int b = tid + i * NT;
        if (B_BLOCKS % NT == 0 || b < B_BLOCKS) {
          const int nb = b % (BN / E), kb = b / (BN / E);
          u32x4 t[E];
          if (ELT == 2)
            transpose8x8_b16(rb[i], t);
          else
            transpose16x16_b8(rb[i], t);
#pragma unroll
          for (int c = 0; c < E; ++c)
            *reinterpret_cast<u32x4 *>(bs + lds_off(nb * E + c, kb, NCH)) = t[c];
        }
      }
      if (SCALED && tid < BM)
        Ss[buf * BM + tid] = rs;
    };

    // One MFMA sub-step (KM elements of K) over the wave's tile.
    auto substep = [&](const uint8_t *as, const uint8_t *bs, int ks, Acc (&dst)[FM][FN]) {
      Frag<CPL> a[FM], b[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int c = 0; c < CPL; ++c)
          a[i].v[c] = *reinterpret_cast<const u32x4 *>(
              as + lds_off(wm * WTM + i * 32 + (lane & 31),
                           ks * 2 * CPL + (lane >> 5) * CPL + c, NCH));
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int c = 0; c < CPL; ++c)
          b[j].v[c] = *reinterpret_cast<const u32x4 *>(
              bs + lds_off(wn * WTN + j * 32 + (lane & 31),
                           ks * 2 * CPL + (lane >> 5) * CPL + c, NCH));
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          dst[i][j] = mfma(T(), a[i], b[j], dst[i][j]);
    };

    // Block-scale epilogue of one K step: acc += (part * sa[m][kb]) * sb[kb][n/128].
    auto scale_add = [&](int buf, int kt, Acc (&part)[FM][FN]) {
      const float *ss = Ss + buf * BM;
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        float sr[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float4 s4 = *reinterpret_cast<const float4 *>(
              ss + wm * WTM + i * 32 + 8 * q + 4 * (lane >> 5));
          sr[4 * q + 0] = s4.x;
          sr[4 * q + 1] = s4.y;
          sr[4 * q + 2] = s4.z;
          sr[4 * q + 3] = s4.w;
        }
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int64_t nblk = (n0 + wn * WTN + j * 32) >> 7;
          float sbv = 0.f;
          if (!MASK_MN || nblk * 128 < p.N)
            sbv = p.sb[(int64_t)kt * p.sb_ld + nblk];
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            // No FMA contraction: the fp32 sequence acc + (part * sa) * sb,
            // each operation rounded.
#pragma clang fp contract(off)
            acc[i][j][r] = acc[i][j][r] + (part[i][j][r] * sr[r]) * sbv;
          }
        }
      }
    };

    // A full K step from LDS buffer `buf` (all KS sub-steps, no branches).
    auto compute_full = [&](int buf, int kt) {
      const uint8_t *as = As + buf * A_BYTES;
      const uint8_t *bs = Bs + buf * B_BYTES;
      if constexpr (SCALED) {
        Acc part[FM][FN];
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r)
              part[i][j][r] = 0;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
          substep(as, bs, ks, part);
        scale_add(buf, kt, part);
      } else {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
          substep(as, bs, ks, acc);
      }
    };

    // The peeled last step: only the sub-steps that reach k < K.
    auto compute_tail = [&](int buf, int kt, int nks) {
      const uint8_t *as = As + buf * A_BYTES;
      const uint8_t *bs = Bs + buf * B_BYTES;
      if constexpr (SCALED) {
        Acc part[FM][FN];
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r)
              part[i][j][r] = 0;
        for (int ks = 0; ks < nks; ++ks)
          substep(as, bs, ks, part);
        scale_add(buf, kt, part);
      } else {
        for (int ks = 0; ks < nks; ++ks)
          substep(as, bs, ks, acc);
      }
    };

    // K loop in LoopSplit form: k_main_steps unmasked steps, then the masked
    // steps (one after a split; all of them with splitting disabled), the last
    // of which issues only last_ks sub-steps.
    const int nmain = p.k_main_steps;
    const int total = nmain + p.k_masked_steps;
    int kt = 0;
    if (nmain > 0) {
      load(0, Unmasked());
      store(0);
      __syncthreads();
      for (; kt < nmain - 1; ++kt) { // branch-free main loop
        load(kt + 1, Unmasked());
        compute_full(kt & 1, kt);
        store((kt + 1) & 1);
        __syncthreads();
      }
      if (total > nmain) { // last main step overlaps the first masked load
        load(kt + 1, Masked());
        compute_full(kt & 1, kt);
        store((kt + 1) & 1);
        __syncthreads();
      } else {
        compute_full(kt & 1, kt);
      }
      ++kt;
    } else if (total > 0) {
      load(0, Masked());
      store(0);
      __syncthreads();
    }
    for (; kt < total; ++kt) { // masked steps
      const bool has_next = kt + 1 < total;
      if (has_next)
        load(kt + 1, Masked());
      if (has_next) {
        compute_full(kt & 1, kt);
        store((kt + 1) & 1);
        __syncthreads();
      } else {
        compute_tail(kt & 1, kt, p.last_ks);
      }
    }

    // Epilogue.  Accumulator register r of lane l in a 32x32 block holds
    // row 8*(r/4) + 4*(l/32) + r%4, column l%32.
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int64_t col = n0 + wn * WTN + j * 32 + (lane & 31);
        float sbc = 1.f;
        if (EPI == EPI_ROWCOL_BF16)
          sbc = (!MASK_MN || col < p.N) ? p.sb[col] : 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t row =
              m0 + wm * WTM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          if (MASK_MN && (row >= p.M || col >= p.N))
            continue;
          const int64_t off = row * p.ldc + col;
          if (EPI == EPI_F32 || EPI == EPI_BLOCK128_F32) {
            float *c = reinterpret_cast<float *>(p.C) + off;
            *c = p.accumulate ? *c + (float)acc[i][j][r] : (float)acc[i][j][r];
          } else if (EPI == EPI_BF16 || EPI == EPI_BLOCK128_BF16) {
            reinterpret_cast<uint16_t *>(p.C)[off] = f32_to_bf16_rne((float)acc[i][j][r]);
          } else if (EPI == EPI_F16) {
            reinterpret_cast<uint16_t *>(p.C)[off] = f32_to_f16_rne((float)acc[i][j][r]);
          } else if (EPI == EPI_I32) {
            int32_t *c = reinterpret_cast<int32_t *>(p.C) + off;
            *c = p.accumulate ? *c + (int32_t)acc[i][j][r] : (int32_t)acc[i][j][r];
          } else { // EPI_ROWCOL_BF16
            const float v = ((float)acc[i][j][r] * p.sa[row]) * sbc;
            reinterpret_cast<uint16_t *>(p.C)[off] = f32_to_bf16_rne(v);
          }
        }
      }
  }
};

template <int OP, int BM, int BN, int BK, int WM, int WN, int EPI>
__global__ void __launch_bounds__(WM * WN * 64, 1)
    gemm_tile_kernel(GemmArgs p) {
  typedef GemmTile<OP, BM, BN, BK, WM, WN, EPI> G;
  extern __shared__ __attribute__((aligned(16))) uint8_t tx_smem[];
  int tm, tn;
  tile_coords(p, tm, tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  if (m0 + BM <= p.M && n0 + BN <= p.N)
    G::template run<false>(p, tx_smem, m0, n0);
  else
    G::template run<true>(p, tx_smem, m0, n0);
}

} // namespace txk
