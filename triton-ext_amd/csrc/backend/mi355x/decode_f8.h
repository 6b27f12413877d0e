// fp8 small-M dot (decode shape) for gfx950, B streamed once through a ring
// shared by the workgroup's waves:
//   unscaled: fp8 x fp8 (e4m3 / e5m2 in any mix), C = sum or C += sum in fp32;
//   SCALED:   e4m3 x e4m3 with 1 x 128 A-group and 128 x 128 B-block scales
//             (the block-scaled fp8 dot): C = sum_kb part_kb * (sa[m][kb] *
//             sb[kb][n / 128]), part_kb the fp32 sum over K block kb, C in
//             bf16 (rounded to nearest even) or fp32;
// with A [M,K] (M <= 64) and B [K,N] row-major.  (An int8 form of this
// kernel, bit-identical to decode_i8.h, measured no faster for W8A8: 18.2 us
// at M = 16 against 18.0-18.4, 23.6 at M = 64 against the row kernel's
// 22.0.)
//
// The layout follows decode16.h with 8-bit elements:
//  * A workgroup owns a strip of 128 columns (128-byte rows of B), the slice
//    of SR = 16 ceil(M / 16) rows and a range of K (split-K).  Batches of 128
//    K rows (16 KiB of B, one K block of the block-scaled dot) and the
//    slice's A rows of the batch go through one LDS ring shared by the 4
//    waves: each wave issues 4 of B's 16 direct-to-LDS loads (non-temporal)
//    and its A rows (8 rows x 128 bytes a load), waits for its own loads and
//    one s_barrier per batch publishes the batch and frees the slot read one
//    batch earlier.
//  * Wave w owns columns 32 w .. 32 w + 31 (two 16-column blocks) for every
//    row of the slice.  Per 16 x 16 block and batch one
//    v_mfma_f32_16x16x128_f8f6f4, with the roles swapped (MFMA A := B columns, MFMA B := A rows):
//    lane l holds row 16 t + l % 16 at the 4 consecutive columns
//    16 j + 4 (l / 16) .. +3.  A lane's operand bytes are K = 32 (l / 16) ..
//    +31 of the batch for both operands (the same permutation of K on both
//    sides, which the dot does not see).
//  * B rows: 16-byte chunk c of row k at c ^ (k & 7); ds_read_b64_tr_b8 hands
//    each lane 8 K-consecutive bytes of one column (within a 16-lane group,
//    lane i gets byte i % 8 of the words read by group lanes 2 r + i / 8),
//    four reads a block.  A rows: chunk c of row r at c ^ ((r >> 1) & 7), so
//    the 16 rows one quarter-wave reads with ds_read_b128 fall in 16 bank
//    groups.
//  * Block scales: per batch, wave 0 stages the slice's sa[.][kb]
//    and wave 1 sb[kb][strip] into the slot by 4-byte direct loads (waves 2
//    and 3 issue the same load of the zero chunk, so every wave counts the
//    same loads); each block's product comes from a fresh MFMA and is added
//    as acc = fma(part, sa * sb, acc).
//  * Split-K: decode_i8.h's exchange (SC1 stores of the partial, an arrival
//    counter per strip that the last arrival resets, the last arrival
//    gathers), fp32 partials in lane order (1 KiB per wave, row tile and
//    column block), added in split order, so the result does not depend on
//    which split arrives last.
//
// K loop in LoopSplit form: batches below k_main_batches load unmasked; the
// rest send B rows >= K, B chunks at or past N and A rows >= M to the
// zero-filled chunk.  An A chunk that crosses K is loaded whole and its bytes
// past K are zeroed in registers (an fp8 NaN code in the padding times B's
// zero rows would be NaN).
//
// BT: B stored K-major ([N][K] row-major, row stride ldb: q . k^T with k
// row-major, or a weight kept [out][in]).  The strip's 128 rows of that
// storage are staged like A's rows (128 bytes of a batch each, chunk c at
// c ^ ((row >> 1) & 7)) and a column block's fragment is read like an A tile
// (ds_read_b128 of chunks 2 G and 2 G + 1), so a lane holds the same K bytes
// of B as of A.  B's chunk that crosses K is loaded whole and zeroed in
// registers like A's.  Each strip starts its split's batches at its own batch
// (strip mod the split's batch count), so the workgroups running at once read
// B's rows at different K offsets.  I8 (with BT only): int8 x int8, int32
// sums, C = sum or C += sum, or the W8A8 epilogue (rowcol: row x column
// scales, bf16 C, as decode_i8.h rounds it); per 16 x 16 block and batch two
// v_mfma_i32_16x16x64_i8 on the same fragments (K bytes 32 G .. +15, then
// +16 .. +31 of each lane), int32 partials, exact in any order.
#pragma once

#include <type_traits>

#include "decode16.h"

namespace txk {

constexpr int kDec8StripN = 128;  // columns: 128-byte rows of B
constexpr int kDec8BatchK = 128;  // K rows a batch (one K block)
constexpr int kDec8MaxM = 64;

struct DecodeF8Args {
  const uint8_t *A;
  const uint8_t *B;
  void *C;
  const float *sa;   // SCALED: [M][sa_ld]
  const float *sb;   // SCALED: [ceil(K / 128)][sb_ld]
  int32_t c_f32;     // fp32 C (else bf16)
  int32_t acc_c;     // fp32 / int32 C: add the sums to C's contents (tl.dot's acc)
  int32_t rowcol;    // I8: W8A8, C = bf16((float(sum) * sa[m]) * sb[n]) (else int32 C)
  int32_t M, N, K;
  int64_t lda, ldb, ldc;
  int32_t sa_ld, sb_ld;
  int32_t ksplit;
  int32_t batches_per_split;
  int32_t k_main_batches;
  float *partials;    // [ksplit][strips][4 waves][SR / 16][2][64 lanes][4] fp32
  uint32_t *counters; // [strips]
};

__host__ __device__ constexpr int64_t decode_f8_split_bytes(int64_t strips, int sr) {
  return strips * sr * kDec8StripN * 4;
}

template <int SR, bool SCALED> struct DecodeF8Cfg {
  static constexpr int T = SR / 16;
  static constexpr int A_LOADS = (SR + 31) / 32;            // per wave: 8 rows a load
  static constexpr int A_OFF = kDec8BatchK * kDec8StripN;   // B's 16 KiB first
  static constexpr int SCL_OFF = A_OFF + kDecodeWaves * A_LOADS * 1024;
  static constexpr int SLOT = SCL_OFF + (SCALED ? 1024 : 0); // 256 bytes of scales a wave
  static constexpr int S = 158 * 1024 / SLOT > 8 ? 8 : 158 * 1024 / SLOT;
  static constexpr int VPB = 4 + A_LOADS + (SCALED ? 1 : 0);
  static_assert(SR == 16 || SR == 32 || SR == 48 || SR == 64, "slices of 16 .. 64 rows");
  static_assert(S >= 3 && (S - 2) * VPB <= 63, "ring depth; vmcnt is 6 bits");
};

// The wave's operands of one batch: the two column blocks' B fragments (four
// transposed reads each, at b0 / b1 + 1 KiB q) and the T row tiles' A
// fragments (two 16-byte reads each, at a0 and a0 ^ 16, +2 KiB per tile),
// waiting for them before the block ends.  Outputs are early-clobber: a
// read lands while later reads of the block still use their address registers.
#define TX_D8_TR                                                                           \
  "ds_read_b64_tr_b8 %0, %[b0]\n\tds_read_b64_tr_b8 %1, %[b0] offset:1024\n\t"             \
  "ds_read_b64_tr_b8 %2, %[b0] offset:2048\n\tds_read_b64_tr_b8 %3, %[b0] offset:3072\n\t" \
  "ds_read_b64_tr_b8 %4, %[b1]\n\tds_read_b64_tr_b8 %5, %[b1] offset:1024\n\t"             \
  "ds_read_b64_tr_b8 %6, %[b1] offset:2048\n\tds_read_b64_tr_b8 %7, %[b1] offset:3072\n\t"
#define TX_D8_OUT                                                                         \
  "=&v"(bq[0][0]), "=&v"(bq[0][1]), "=&v"(bq[0][2]), "=&v"(bq[0][3]), "=&v"(bq[1][0]),        \
      "=&v"(bq[1][1]), "=&v"(bq[1][2]), "=&v"(bq[1][3])
#define TX_D8_IN [b0] "v"(b0), [b1] "v"(b1), [a0] "v"(a0), [a1] "v"(a1)
template <int T>
__device__ __forceinline__ void dec8_read(uint32_t b0, uint32_t b1, uint32_t a0, uint32_t a1,
                                          v2i_t (&bq)[2][4], i32x4_t (&a)[T][2]) {
  if constexpr (T == 1)
    asm volatile(TX_D8_TR "ds_read_b128 %8, %[a0]\n\tds_read_b128 %9, %[a1]\n\t"
                          "s_waitcnt lgkmcnt(0)"
                 : TX_D8_OUT, "=&v"(a[0][0]), "=&v"(a[0][1])
                 : TX_D8_IN
                 : "memory");
  else if constexpr (T == 2)
    asm volatile(TX_D8_TR "ds_read_b128 %8, %[a0]\n\tds_read_b128 %9, %[a1]\n\t"
                          "ds_read_b128 %10, %[a0] offset:2048\n\tds_read_b128 %11, %[a1] offset:2048\n\t"
                          "s_waitcnt lgkmcnt(0)"
                 : TX_D8_OUT, "=&v"(a[0][0]), "=&v"(a[0][1]), "=&v"(a[1][0]), "=&v"(a[1][1])
                 : TX_D8_IN
                 : "memory");
  else if constexpr (T == 3)
    asm volatile(TX_D8_TR "ds_read_b128 %8, %[a0]\n\tds_read_b128 %9, %[a1]\n\t"
                          "ds_read_b128 %10, %[a0] offset:2048\n\tds_read_b128 %11, %[a1] offset:2048\n\t"
                          "ds_read_b128 %12, %[a0] offset:4096\n\tds_read_b128 %13, %[a1] offset:4096\n\t"
                          "s_waitcnt lgkmcnt(0)"
                 : TX_D8_OUT, "=&v"(a[0][0]), "=&v"(a[0][1]), "=&v"(a[1][0]), "=&v"(a[1][1]),
                   "=&v"(a[2][0]), "=&v"(a[2][1])
                 : TX_D8_IN
                 : "memory");
  else
    asm volatile(TX_D8_TR "ds_read_b128 %8, %[a0]\n\tds_read_b128 %9, %[a1]\n\t"
                          "ds_read_b128 %10, %[a0] offset:2048\n\tds_read_b128 %11, %[a1] offset:2048\n\t"
                          "ds_read_b128 %12, %[a0] offset:4096\n\tds_read_b128 %13, %[a1] offset:4096\n\t"
                          "ds_read_b128 %14, %[a0] offset:6144\n\tds_read_b128 %15, %[a1] offset:6144\n\t"
                          "s_waitcnt lgkmcnt(0)"
                 : TX_D8_OUT, "=&v"(a[0][0]), "=&v"(a[0][1]), "=&v"(a[1][0]), "=&v"(a[1][1]),
                   "=&v"(a[2][0]), "=&v"(a[2][1]), "=&v"(a[3][0]), "=&v"(a[3][1])
                 : TX_D8_IN
                 : "memory");
}
#undef TX_D8_IN
#undef TX_D8_OUT
#undef TX_D8_TR

// The same with B K-major: each column block's fragment is two 16-byte reads
// (at b0 / b1 and their ^ 16, chunks 2 G and 2 G + 1), like A's, which are
// at a0 and a0 ^ 16, +2 KiB per tile.
#define TX_D8K_T(t, off)                                                                   \
  "ds_read_b128 %[x0" #t "], %[a0] offset:" #off "\n\tds_read_b128 %[x1" #t "], %[a1] offset:" #off \
  "\n\t"
#define TX_D8K_O(t) [x0##t] "=&v"(a[t][0]), [x1##t] "=&v"(a[t][1])
#define TX_D8K_HEAD                                                                        \
  "ds_read_b128 %[y00], %[b0]\n\tds_read_b128 %[y01], %[b0x]\n\t"                           \
  "ds_read_b128 %[y10], %[b1]\n\tds_read_b128 %[y11], %[b1x]\n\t"
#define TX_D8K_BO                                                                          \
  [y00] "=&v"(bk[0][0]), [y01] "=&v"(bk[0][1]), [y10] "=&v"(bk[1][0]), [y11] "=&v"(bk[1][1])
#define TX_D8K_IN                                                                          \
  [b0] "v"(b0), [b0x] "v"(b0 ^ 16u), [b1] "v"(b1), [b1x] "v"(b1 ^ 16u), [a0] "v"(a0),         \
      [a1] "v"(a0 ^ 16u)
template <int T>
__device__ __forceinline__ void dec8_read_kmajor(uint32_t b0, uint32_t b1, uint32_t a0,
                                                 i32x4_t (&bk)[2][2], i32x4_t (&a)[T][2]) {
  if constexpr (T == 1)
    asm volatile(TX_D8K_HEAD TX_D8K_T(0, 0) "s_waitcnt lgkmcnt(0)"
                 : TX_D8K_BO, TX_D8K_O(0)
                 : TX_D8K_IN
                 : "memory");
  else if constexpr (T == 2)
    asm volatile(TX_D8K_HEAD TX_D8K_T(0, 0) TX_D8K_T(1, 2048) "s_waitcnt lgkmcnt(0)"
                 : TX_D8K_BO, TX_D8K_O(0), TX_D8K_O(1)
                 : TX_D8K_IN
                 : "memory");
  else if constexpr (T == 3)
    asm volatile(TX_D8K_HEAD TX_D8K_T(0, 0) TX_D8K_T(1, 2048) TX_D8K_T(2, 4096)
                 "s_waitcnt lgkmcnt(0)"
                 : TX_D8K_BO, TX_D8K_O(0), TX_D8K_O(1), TX_D8K_O(2)
                 : TX_D8K_IN
                 : "memory");
  else
    asm volatile(TX_D8K_HEAD TX_D8K_T(0, 0) TX_D8K_T(1, 2048) TX_D8K_T(2, 4096)
                 TX_D8K_T(3, 6144) "s_waitcnt lgkmcnt(0)"
                 : TX_D8K_BO, TX_D8K_O(0), TX_D8K_O(1), TX_D8K_O(2), TX_D8K_O(3)
                 : TX_D8K_IN
                 : "memory");
}
#undef TX_D8K_IN
#undef TX_D8K_BO
#undef TX_D8K_HEAD
#undef TX_D8K_O
#undef TX_D8K_T

// FA, FB: the MFMA format codes of A and B (0 e4m3, 1 e5m2); SCALED takes
// e4m3 x e4m3 with block scales.  BT: B K-major; I8: int8 -> int32 (BT only).
template <int SR, bool SCALED, int FA = 0, int FB = 0, bool BT = false, bool I8 = false>
__global__ void __launch_bounds__(kDecodeWaves * 64, 1) decode_f8_kernel(DecodeF8Args p) {
  static_assert(!SCALED || (FA == 0 && FB == 0), "block scales take e4m3 operands");
  static_assert(!I8 || (BT && FA == 0 && FB == 0), "int8: the K-major form");
  typedef DecodeF8Cfg<SR, SCALED> Cfg;
  constexpr int S = Cfg::S, SLOT = Cfg::SLOT, T = Cfg::T;
  typedef std::conditional_t<I8, i32x4_t, f32x4_t> Acc;
  __shared__ __attribute__((aligned(1024))) uint8_t ring[S * SLOT];
  __shared__ uint32_t last_flag;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = lane >> 4, L = lane & 15;
  const int strips = (p.N + kDec8StripN - 1) / kDec8StripN;
  const int strip = blockIdx.x % strips, split = blockIdx.x / strips;
  const int64_t n0 = (int64_t)strip * kDec8StripN;
  const bool n_edge = n0 + kDec8StripN > p.N;

  const int total_batches = (p.K + kDec8BatchK - 1) / kDec8BatchK;
  const int b_begin = split * p.batches_per_split;
  int b_end = b_begin + p.batches_per_split;
  if (b_end > total_batches)
    b_end = total_batches;
  const int nb = b_end > b_begin ? b_end - b_begin : 0;
  const int rot = BT && nb > 0 ? strip % nb : 0; // K-major B: the strip's first batch
  auto batch = [&](int i) { // the split's i-th batch to run (i < nb)
    if constexpr (!BT)
      return b_begin + i;
    const int j = i + rot;
    return b_begin + (j >= nb ? j - nb : j);
  };

  // Loads of the split's batch i into `slot`: B rows 32 wave .. +31 (load u:
  // rows 8 q .. +7, q = 4 wave + u, lane l' fetching chunk (l' % 8) ^ (row &
  // 7) of row 8 q + l' / 8; K-major B: storage rows n0 + 8 q .. +7, lane l'
  // fetching chunk (l' % 8) ^ ((row >> 1) & 7), as for A), A rows 8 q .. +7
  // (q = A_LOADS wave + u, lane l' fetching chunk (l' % 8) ^ ((row >> 1) &
  // 7)), and with block scales wave 0's sa[row][kb] (lane = row) and wave 1's
  // sb[kb][strip] (every lane).  For i >= nb every load reads the zero chunk,
  // so each step issues the same loads.
  auto issue = [&](int i, uint8_t *slot) {
    const bool live = i < nb;
    const int b = live ? batch(i) : b_begin + i;
    const int64_t k0 = (int64_t)b * kDec8BatchK;
    const bool mask = !live || n_edge || b >= p.k_main_batches;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int q = 4 * wave + u;
      const int row = 8 * q + (lane >> 3);
      const void *src;
      if constexpr (BT) {
        const int c = (lane & 7) ^ ((row >> 1) & 7);
        const int64_t n = n0 + row, k = k0 + 16 * c;
        src = p.B + n * p.ldb + k;
        if (mask && (!live || n >= p.N || k >= p.K))
          src = tx_zero_chunk;
      } else {
        const int c = (lane & 7) ^ (row & 7);
        const int64_t k = k0 + row, n = n0 + 16 * c;
        src = p.B + k * p.ldb + n;
        if (mask && (!live || k >= p.K || n >= p.N))
          src = tx_zero_chunk;
      }
      dma16_stream(src, (lds_void *)(slot + q * 1024)); // B is read once
    }
#pragma unroll
    for (int u = 0; u < Cfg::A_LOADS; ++u) {
      const int q = Cfg::A_LOADS * wave + u;
      const int r = 8 * q + (lane >> 3);
      const int c = (lane & 7) ^ ((r >> 1) & 7);
      const int64_t k = k0 + 16 * c;
      const void *src = p.A + (int64_t)r * p.lda + k;
      if (!live || r >= p.M || (b >= p.k_main_batches && k >= p.K))
        src = tx_zero_chunk;
      dma16(src, (lds_void *)(slot + Cfg::A_OFF + q * 1024)); // A: re-read by every strip
    }
    if constexpr (SCALED) {
      const void *src = tx_zero_chunk;
      if (live && wave == 0 && lane < p.M)
        src = p.sa + (int64_t)lane * p.sa_ld + b;
      else if (live && wave == 1)
        src = p.sb + (int64_t)b * p.sb_ld + strip;
      __builtin_amdgcn_global_load_lds(src, (lds_void *)(slot + Cfg::SCL_OFF + 256 * wave), 4,
                                       0, 0);
    }
  };

  Acc acc[T][2];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
      acc[t][jj] = Acc{0, 0, 0, 0};

  // Per-lane LDS offsets within a slot.  B, column block j = 2 wave + jj,
  // read q: row 32 G + 8 q + L / 2 (row & 7 = L / 2), chunk j, byte 8 (L % 2):
  // +1 KiB per read.  A, tile t: row 16 t + L ((row >> 1) & 7 = L / 2),
  // chunks 2 G and 2 G + 1 (the second at the first ^ 16): +2 KiB per tile.
  // K-major B, block j: storage row 16 j + L, chunks 2 G and 2 G + 1, like A.
  uint32_t b_off[2];
#pragma unroll
  for (int jj = 0; jj < 2; ++jj) {
    const int j = 2 * wave + jj;
    b_off[jj] = BT ? (16 * j + L) * 128 + (((2 * G) ^ (L >> 1)) << 4)
                   : (32 * G + (L >> 1)) * 128 + ((j ^ (L >> 1)) << 4) + 8 * (L & 1);
  }
  const uint32_t a_off = Cfg::A_OFF + L * 128 + (((2 * G) ^ (L >> 1)) << 4);

  // operand formats FB (MFMA A := B columns) and FA; no hardware scales
  auto mma = [&](const i32x8_t &bcol, const i32x8_t &arow, f32x4_t c) -> f32x4_t {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bcol, arow, c, FB, FA, 0, 0, 0, 0);
  };

  auto consume = [&](const uint8_t *slot, int i) {
    const uint32_t base = lds_addr(slot);
    i32x4_t bk[2][2]; // column block jj's fragment (K-major B): chunks 2 G, 2 G + 1
    v2i_t bq[2][4];
    i32x4_t a[T][2];
    if constexpr (BT)
      dec8_read_kmajor<T>(base + b_off[0], base + b_off[1], base + a_off, bk, a);
    else
      dec8_read<T>(base + b_off[0], base + b_off[1], base + a_off, (base + a_off) ^ 16u, bq, a);
    const int b = batch(i);
    if (b >= p.k_main_batches) { // the K tail: bytes of A (and K-major B) at or past K
      const int64_t k = (int64_t)b * kDec8BatchK + 32 * G;
#pragma unroll
      for (int t = 0; t < T; ++t) {
        a[t][0] = dec8_mask_k(a[t][0], k, p.K);
        a[t][1] = dec8_mask_k(a[t][1], k + 16, p.K);
      }
      if constexpr (BT) {
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          bk[jj][0] = dec8_mask_k(bk[jj][0], k, p.K);
          bk[jj][1] = dec8_mask_k(bk[jj][1], k + 16, p.K);
        }
      }
    }
    float s_row[T], s_col = 0.f;
    if constexpr (SCALED) {
      const uint32_t sb_addr = base + Cfg::SCL_OFF + 256;
      float v;
      asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=&v"(v) : "v"(sb_addr) : "memory");
      s_col = v;
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const uint32_t sa_addr = base + Cfg::SCL_OFF + 4 * (16 * t + L);
        asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=&v"(v) : "v"(sa_addr) : "memory");
        s_row[t] = v * s_col;
      }
    }
    if constexpr (I8) { // two K steps of 64: bytes 32 G .. +15, then +16 .. +31; a step's
                        // 2 T products are independent of each other
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
#pragma unroll
          for (int t = 0; t < T; ++t)
            acc[t][jj] = mfma_i8_16(bk[jj][h], a[t][h], acc[t][jj]);
    } else {
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const i32x8_t bcol =
            BT ? i32x8_t{bk[jj][0][0], bk[jj][0][1], bk[jj][0][2], bk[jj][0][3], bk[jj][1][0],
                         bk[jj][1][1], bk[jj][1][2], bk[jj][1][3]}
               : i32x8_t{bq[jj][0].x, bq[jj][0].y, bq[jj][1].x, bq[jj][1].y,
                         bq[jj][2].x, bq[jj][2].y, bq[jj][3].x, bq[jj][3].y};
#pragma unroll
        for (int t = 0; t < T; ++t) {
          const i32x8_t arow = {a[t][0][0], a[t][0][1], a[t][0][2], a[t][0][3],
                                a[t][1][0], a[t][1][1], a[t][1][2], a[t][1][3]};
          if constexpr (SCALED) {
            const f32x4_t part = mma(bcol, arow, f32x4_t{0, 0, 0, 0});
#pragma unroll
            for (int r = 0; r < 4; ++r)
              acc[t][jj][r] = __builtin_fmaf(part[r], s_row[t], acc[t][jj][r]);
          } else {
            acc[t][jj] = mma(bcol, arow, acc[t][jj]);
          }
        }
      }
    }
  };

  // Prologue: S - 1 batches in flight; batch i uses slot i % S.
#pragma unroll
  for (int s = 0; s < S - 1; ++s)
    issue(s, ring + s * SLOT);
  // Main loop (decode16.h's): wait for this wave's loads of batch i, barrier,
  // issue batch i + S - 1 into the slot read at batch i - 1, MFMAs of batch i.
  for (int i0 = 0;; i0 += S) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int i = i0 + s;
      if (i >= nb)
        goto k_loop_done;
      wait_vmcnt<(S - 2) * Cfg::VPB>();
      asm volatile("s_barrier" ::: "memory");
      issue(i + S - 1, ring + ((s + S - 1) % S) * SLOT);
      consume(ring + s * SLOT, i);
    }
  }
k_loop_done:
  __builtin_amdgcn_s_waitcnt(0); // the zero-chunk loads past nb have landed

  // C for this lane: row 16 t + L, columns n0 + 16 (2 wave + jj) + 4 G .. +3.
  auto epilogue = [&](const Acc (&sum)[T][2]) {
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int64_t col = n0 + 16 * (2 * wave + jj) + 4 * G;
      if (col >= p.N)
        continue;
      const bool whole = col + 4 <= p.N;
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const int m = 16 * t + L;
        if (m >= p.M)
          continue;
        if constexpr (I8) {
          if (p.rowcol) { // W8A8: bf16((float(sum) * sa[m]) * sb[n]), nearest even
            const float sam = p.sa[m];
            float f[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
#pragma clang fp contract(off)
              f[r] = ((float)sum[t][jj][r] * sam) * p.sb[col + r < p.N ? col + r : 0];
            }
            uint16_t *c = static_cast<uint16_t *>(p.C) + (int64_t)m * p.ldc + col;
            if (whole) {
              uint2 w;
              w.x = pk_bf16_rne(f[0], f[1]);
              w.y = pk_bf16_rne(f[2], f[3]);
              *reinterpret_cast<uint2 *>(c) = w;
            } else {
#pragma unroll
              for (int r = 0; r < 4; ++r)
                if (col + r < p.N)
                  c[r] = f32_to_bf16_rne(f[r]);
            }
          } else { // int32 C
            int32_t *c = static_cast<int32_t *>(p.C) + (int64_t)m * p.ldc + col;
            if (whole) {
              i32x4_t v = sum[t][jj];
              if (p.acc_c)
                v += *reinterpret_cast<const i32x4_t *>(c);
              *reinterpret_cast<i32x4_t *>(c) = v;
            } else {
#pragma unroll
              for (int r = 0; r < 4; ++r)
                if (col + r < p.N)
                  c[r] = p.acc_c ? c[r] + sum[t][jj][r] : sum[t][jj][r];
            }
          }
        } else if (p.c_f32) { // fp32 C
          float *c = static_cast<float *>(p.C) + (int64_t)m * p.ldc + col;
          if (whole) {
            f32x4_t v = sum[t][jj];
            if (p.acc_c)
              v += *reinterpret_cast<const f32x4_t *>(c);
            *reinterpret_cast<f32x4_t *>(c) = v;
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (col + r < p.N)
                c[r] = p.acc_c ? c[r] + sum[t][jj][r] : sum[t][jj][r];
          }
        } else { // bf16 C, rounded to nearest even
          const float f[4] = {sum[t][jj][0], sum[t][jj][1], sum[t][jj][2], sum[t][jj][3]};
          uint16_t *c = static_cast<uint16_t *>(p.C) + (int64_t)m * p.ldc + col;
          if (whole) {
            uint2 w;
            w.x = pk_bf16_rne(f[0], f[1]);
            w.y = pk_bf16_rne(f[2], f[3]);
            *reinterpret_cast<uint2 *>(c) = w;
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (col + r < p.N)
                c[r] = f32_to_bf16_rne(f[r]);
          }
        }
      }
    }
  };
  if (p.ksplit == 1) {
    epilogue(acc);
    return;
  }

  // Split-K exchange (decode16.h's), partials in lane order: block
  // ((strip * 4 + wave) * T + t) * 2 + jj of 1 KiB.
  constexpr int kSC1 = 16;
  const int64_t split_bytes = decode_f8_split_bytes(strips, SR);
  auto part_rsrc = [&](int q) {
    return __builtin_amdgcn_make_buffer_rsrc(
        reinterpret_cast<uint8_t *>(p.partials) + (int64_t)q * split_bytes, 0, (int)split_bytes,
        0x00020000);
  };
  const int blk0 = (strip * kDecodeWaves + wave) * T * 2;
  {
    const auto mine = part_rsrc(split);
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4i_t, acc[t][jj]), mine,
                                               ((blk0 + 2 * t + jj) << 10) + 16 * lane, 0, kSC1);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    uint32_t *const ctr = &p.counters[strip];
    const uint32_t old =
        __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = old + 1 == (uint32_t)p.ksplit;
    if (last) // every split has arrived: none touches the counter again
      __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *reinterpret_cast<volatile uint32_t *>(&last_flag) = last;
  }
  __syncthreads();
  if (!*reinterpret_cast<volatile uint32_t *>(&last_flag))
    return;
  // Last arrival: partial 0 + partial 1 + .. in split order, its own from
  // registers; NQ splits' loads in flight before any is used.
  Acc sum[T][2];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
      sum[t][jj] = Acc{0, 0, 0, 0};
  constexpr int NQ = 4 / T > 1 ? 4 / T : 1;
  for (int q0 = 0; q0 < p.ksplit; q0 += NQ) {
    v4i_t v[NQ][T][2];
#pragma unroll
    for (int qq = 0; qq < NQ; ++qq)
      if (q0 + qq < p.ksplit && q0 + qq != split) {
        const auto r = part_rsrc(q0 + qq);
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
          for (int jj = 0; jj < 2; ++jj)
            v[qq][t][jj] = __builtin_amdgcn_raw_buffer_load_b128(
                r, ((blk0 + 2 * t + jj) << 10) + 16 * lane, 0, kSC1);
      }
#pragma unroll
    for (int qq = 0; qq < NQ; ++qq)
      if (q0 + qq < p.ksplit)
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
          for (int jj = 0; jj < 2; ++jj)
            sum[t][jj] += q0 + qq == split ? acc[t][jj] : __builtin_bit_cast(Acc, v[qq][t][jj]);
  }
  epilogue(sum);
}

} // namespace txk
