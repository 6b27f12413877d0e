// int8 W8A8 dot for taller decode shapes (64 < M <= 256) on gfx950:
//   C[m][n] = bf16((float(sum_k A[m][k] * B[k][n]) * sa[m]) * sb[n])
// with A int8 [M,K], B int8 [K,N] row-major, int32 accumulation (or the
// int32 sums themselves for an unscaled int8 -> int32 dot): the same job and
// result as decode_i8.h, with the work split the other way.
//
// decode_i8.h gives each workgroup a row slice of at most 64 rows, so past
// M = 64 every 128-column strip of B is streamed once per slice, and its 4
// waves split K.  Here a workgroup owns a slice of 64, 128 or 256 rows (one
// slice covers M when it is as tall), a strip of 128 columns and a range of
// K (split-K); its 4 waves each own a block of the slice's outputs (32 or 64
// rows by all 128 columns, or at 64 rows 32 rows by 64 columns) and all take
// every batch of 128 K rows:
//  * B's batches go through one LDS ring shared by the 4 waves: each wave
//    issues 4 of a batch's 16 direct-to-LDS loads (global_load_lds_dwordx4,
//    non-temporal), waits for its own loads (s_waitcnt vmcnt) and one
//    s_barrier per batch makes the whole batch visible; that barrier also
//    tells every wave that the slot read one batch earlier is free, and the
//    loads of the batch S - 1 ahead go into it.  B is read once per slice.
//  * A goes through the same slots: the slice's rows x 128 bytes of the
//    batch, a quarter loaded by each wave, each load 8 whole 128-byte lines (loads of 16 rows x 64
//    bytes, half lines, measured 2.8 times slower per byte), stored
//    row-major with 16-byte chunk c of row r at c ^ ((r >> 1) & 7), so the
//    16 rows one ds_read_b128 quarter-wave reads sit in 16 bank groups.
//  * B's LDS layout and transposed reads are decode_i8.h's (128-byte rows,
//    chunk c of row r at c ^ (r & 7), ds_read_b64_tr_b8 pairs).
//  * Products 32 x 32 x 32 at a time (v_mfma_i32_32x32x32_i8: at one wave
//    per SIMD it runs at 4.3 POP/s on the chip, v_mfma_i32_16x16x64_i8 at
//    1.6), four K steps a batch, with the MFMA roles swapped (MFMA A := B
//    columns, MFMA B := A rows), so the result is C^T: lane l holds C row
//    32 rb + l%32 of the wave's rows at the 4 consecutive columns
//    32 cb + 8 q + 4 (l/32) .. +3 of its column blocks.  No cross-wave reduction: the waves own disjoint outputs.
//  * The epilogue's scales are staged in LDS by 4-byte direct loads that go
//    out before the first batch.
//  * Split-K: decode_i8.h's exchange (SC1 stores of the int32 partial, an
//    arrival counter per (slice, strip) that the last arrival resets, the
//    last arrival adds the others' partials and applies the epilogue).
//    Partials are kept in lane order: 4 KiB per (wave, rb, cb) block, so
//    every store and load instruction moves 1 KiB of contiguous memory.
//
// K loop in LoopSplit form as in decode_i8.h (for 128-row batches):
// batches below k_main_batches load unmasked; the rest send rows >= K,
// columns >= N and rows of A >= M to the zero-filled chunk.
//
// BT: B stored K-major ([N][K] row-major, row stride ldb: a W8A8 weight kept
// [out][in]).  The strip's 128 storage rows are staged like A's rows (128
// bytes of a batch each, chunk c of row r at c ^ ((r >> 1) & 7)) and a column
// block's operand is read like an A row block (ds_read_b128: lane l gets
// column 32 cb + l%32 at K bytes 32 ks + 16 (l/32) .. +15, the bytes of the A
// operand it meets).  B's chunk that crosses K is loaded whole too, so in the
// tail batch its bytes past K are zeroed in registers (A's junk past K then
// meets zeros).  Each strip starts its split's batches at its own batch
// (strip mod the batch count), so the workgroups running at once read B's
// rows at different K offsets.
#pragma once

#include <type_traits>

#include "decode_i8.h"

namespace txk {

// The row kernel's partials per split: every slice (sr rows) and strip, its
// sr x 128 int32 sums in lane order.
__host__ __device__ constexpr int64_t decode_rows_split_bytes(int slices, int strips, int sr) {
  return (int64_t)slices * strips * sr * kDecodeStripN * 4;
}

constexpr int kRowsBatchK = 128; // K rows per batch: A's rows are whole 128-byte lines
constexpr int kDecodeRowsMaxM = 1024; // row slices of one launch: up to 16 of 64 rows

// SR: rows a slice (64, 128 or 256); S: ring slots, each one batch: B's
// 16 KiB, then the slice's A rows (SR x 128 bytes).  The 4 waves cover the
// slice as WR row groups of WROWS rows by WC column groups: 4 x 1 waves of
// 32 or 64 rows and all 128 columns past 64 rows, 2 x 2 waves of 32 rows and
// 64 columns at 64 (a 32 x 32 MFMA block needs 32 rows).
template <int SR, int S> struct DecodeRowsCfg {
  static constexpr int WC = SR == 64 ? 2 : 1, WR = kDecodeWaves / WC, WROWS = SR / WR;
  static constexpr int R32 = WROWS / 32, NCB = 4 / WC; // 32 x 32 blocks a wave
  static constexpr int A_OFF = kRowsBatchK * kDecodeStripN; // 16 KiB of B
  static constexpr int SLOT = A_OFF + SR * kRowsBatchK;
  static constexpr int B_LOADS = A_OFF / 1024 / kDecodeWaves;          // per wave and batch
  static constexpr int A_LOADS = SR * kRowsBatchK / 1024 / kDecodeWaves; // SR / 4 rows a wave
  static constexpr int VPB = B_LOADS + A_LOADS;
  static_assert(SR == 64 || SR == 128 || SR == 256, "slices of 64, 128 or 256 rows");
  static_assert(S >= 3 && S * SLOT <= 158 * 1024, "ring (and the scales) fit LDS");
  static_assert((S - 2) * VPB <= 63, "vmcnt is 6 bits");
};

// One K step (32 rows, KS of the batch's 4) of operands: the 4 column
// blocks' B fragments (decode_i8.h's tr32_off layout, 4 KiB a step) and the
// wave's R32 A row blocks (a_addr, +4 KiB per 32 rows), waiting for them
// before the asm block ends.  Outputs are early-clobber: a read lands while
// later reads of the block still use their address registers.
#define TX_ROWS_TR(O0, O1, A, B, C, D)                                                      \
  "ds_read_b64_tr_b8 %0, %" #A " offset:" #O0 "\n\tds_read_b64_tr_b8 %1, %" #A " offset:" #O1   \
  "\n\tds_read_b64_tr_b8 %2, %" #B " offset:" #O0 "\n\tds_read_b64_tr_b8 %3, %" #B             \
  " offset:" #O1 "\n\tds_read_b64_tr_b8 %4, %" #C " offset:" #O0                                 \
  "\n\tds_read_b64_tr_b8 %5, %" #C " offset:" #O1 "\n\tds_read_b64_tr_b8 %6, %" #D             \
  " offset:" #O0 "\n\tds_read_b64_tr_b8 %7, %" #D " offset:" #O1 "\n\t"
#define TX_ROWS_OUT8                                                                       \
  "=&v"(lo[0]), "=&v"(hi[0]), "=&v"(lo[1]), "=&v"(hi[1]), "=&v"(lo[2]), "=&v"(hi[2]), "=&v"(lo[3]),   \
      "=&v"(hi[3])
#define TX_ROWS_IN4 "v"(b + off[0]), "v"(b + off[1]), "v"(b + off[2]), "v"(b + off[3])
#define TX_ROWS_K1(O0, O1)                                                                 \
  asm volatile(TX_ROWS_TR(O0, O1, 9, 10, 11, 12) "ds_read_b128 %8, %13\n\ts_waitcnt lgkmcnt(0)"  \
               : TX_ROWS_OUT8, "=&v"(a[0])                                                  \
               : TX_ROWS_IN4, "v"(a_addr)                                                  \
               : "memory")
#define TX_ROWS_H1(O0, O1)                                                                 \
  asm volatile("ds_read_b64_tr_b8 %0, %5 offset:" #O0 "\n\tds_read_b64_tr_b8 %1, %5 offset:" #O1 \
               "\n\tds_read_b64_tr_b8 %2, %6 offset:" #O0 "\n\tds_read_b64_tr_b8 %3, %6 offset:" #O1 \
               "\n\tds_read_b128 %4, %7\n\ts_waitcnt lgkmcnt(0)"                              \
               : "=&v"(lo[0]), "=&v"(hi[0]), "=&v"(lo[1]), "=&v"(hi[1]), "=&v"(a[0])           \
               : "v"(b + off[0]), "v"(b + off[1]), "v"(a_addr)                             \
               : "memory")
#define TX_ROWS_K2(O0, O1)                                                                 \
  asm volatile(TX_ROWS_TR(O0, O1, 10, 11, 12, 13)                                          \
               "ds_read_b128 %8, %14\n\tds_read_b128 %9, %14 offset:4096\n\t"               \
               "s_waitcnt lgkmcnt(0)"                                                      \
               : TX_ROWS_OUT8, "=&v"(a[0]), "=&v"(a[1])                                      \
               : TX_ROWS_IN4, "v"(a_addr)                                                  \
               : "memory")
template <int R32, int NCB, int KS>
__device__ __forceinline__ void rows_read_k32(uint32_t b, const uint32_t (&off)[NCB],
                                              uint32_t a_addr, v2i_t (&lo)[NCB],
                                              v2i_t (&hi)[NCB], i32x4_t (&a)[R32]) {
  static_assert((R32 == 1 || R32 == 2) && (NCB == 4 || (NCB == 2 && R32 == 1)),
                "32 or 64 rows by 128 columns, or 32 rows by 64 columns, a wave");
  if constexpr (NCB == 2) {
    if constexpr (KS == 0) TX_ROWS_H1(0, 1024);
    else if constexpr (KS == 1) TX_ROWS_H1(4096, 5120);
    else if constexpr (KS == 2) TX_ROWS_H1(8192, 9216);
    else TX_ROWS_H1(12288, 13312);
  } else if constexpr (R32 == 1) {
    if constexpr (KS == 0) TX_ROWS_K1(0, 1024);
    else if constexpr (KS == 1) TX_ROWS_K1(4096, 5120);
    else if constexpr (KS == 2) TX_ROWS_K1(8192, 9216);
    else TX_ROWS_K1(12288, 13312);
  } else {
    if constexpr (KS == 0) TX_ROWS_K2(0, 1024);
    else if constexpr (KS == 1) TX_ROWS_K2(4096, 5120);
    else if constexpr (KS == 2) TX_ROWS_K2(8192, 9216);
    else TX_ROWS_K2(12288, 13312);
  }
}
#undef TX_ROWS_K2
#undef TX_ROWS_H1
#undef TX_ROWS_K1
#undef TX_ROWS_IN4
#undef TX_ROWS_OUT8
#undef TX_ROWS_TR

// The same K step with B K-major: the NCB column blocks' operands with
// ds_read_b128 at `bk` (+4 KiB per block) and the R32 A row blocks at `ak`
// (+4 KiB per 32 rows).
#define TX_RK_B(i, off) "ds_read_b128 %[y" #i "], %[bk] offset:" #off "\n\t"
#define TX_RK_A(i, off) "ds_read_b128 %[x" #i "], %[ak] offset:" #off "\n\t"
#define TX_RK_BO(i) [y##i] "=&v"(b[i])
#define TX_RK_AO(i) [x##i] "=&v"(a[i])
#define TX_RK_IN [bk] "v"(bk), [ak] "v"(ak)
template <int R32, int NCB>
__device__ __forceinline__ void rows_read_k32_kmajor(uint32_t bk, uint32_t ak, i32x4_t (&b)[NCB],
                                                     i32x4_t (&a)[R32]) {
  static_assert((R32 == 1 || R32 == 2) && (NCB == 4 || (NCB == 2 && R32 == 1)),
                "32 or 64 rows by 128 columns, or 32 rows by 64 columns, a wave");
  if constexpr (NCB == 2)
    asm volatile(TX_RK_B(0, 0) TX_RK_B(1, 4096) TX_RK_A(0, 0) "s_waitcnt lgkmcnt(0)"
                 : TX_RK_BO(0), TX_RK_BO(1), TX_RK_AO(0)
                 : TX_RK_IN
                 : "memory");
  else if constexpr (R32 == 1)
    asm volatile(TX_RK_B(0, 0) TX_RK_B(1, 4096) TX_RK_B(2, 8192) TX_RK_B(3, 12288)
                 TX_RK_A(0, 0) "s_waitcnt lgkmcnt(0)"
                 : TX_RK_BO(0), TX_RK_BO(1), TX_RK_BO(2), TX_RK_BO(3), TX_RK_AO(0)
                 : TX_RK_IN
                 : "memory");
  else
    asm volatile(TX_RK_B(0, 0) TX_RK_B(1, 4096) TX_RK_B(2, 8192) TX_RK_B(3, 12288)
                 TX_RK_A(0, 0) TX_RK_A(1, 4096) "s_waitcnt lgkmcnt(0)"
                 : TX_RK_BO(0), TX_RK_BO(1), TX_RK_BO(2), TX_RK_BO(3), TX_RK_AO(0), TX_RK_AO(1)
                 : TX_RK_IN
                 : "memory");
}
#undef TX_RK_IN
#undef TX_RK_AO
#undef TX_RK_BO
#undef TX_RK_A
#undef TX_RK_B

template <int SR, int S, bool BT = false>
__global__ void __launch_bounds__(kDecodeWaves * 64, 1) decode_rows_i8_kernel(DecodeArgs p) {
  typedef DecodeRowsCfg<SR, S> Cfg;
  constexpr int SLOT = Cfg::SLOT, WC = Cfg::WC, WROWS = Cfg::WROWS, R32 = Cfg::R32,
                NCB = Cfg::NCB;
  __shared__ __attribute__((aligned(1024))) uint8_t ring[S * SLOT];
  __shared__ uint32_t last_flag;
  // The epilogue's scales: sb of the strip's 128 columns, then 64 sa values
  // per wave (its WROWS rows first).
  __shared__ __attribute__((aligned(16))) float scl[kDecodeStripN + 64 * kDecodeWaves];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Workgroup -> (slice, strip, split), decode_i8.h's order: consecutive
  // workgroups are adjacent strips of one split, and the slices of one
  // (strip, split) go to one XCD (workgroups are dealt to the 8 XCDs
  // round-robin) so they read its B through one L2.
  const int strips = (p.N + kDecodeStripN - 1) / kDecodeStripN;
  const int pairs = strips * p.ksplit;
  int slice = 0, pair = blockIdx.x;
  if (p.slices > 1) {
    if (pairs % 8 == 0) {
      const int jj = blockIdx.x / 8;
      slice = jj % p.slices;
      pair = 8 * (jj / p.slices) + blockIdx.x % 8;
    } else {
      slice = blockIdx.x % p.slices;
      pair = blockIdx.x / p.slices;
    }
  }
  const int strip = pair % strips, split = pair / strips;
  const int64_t n0 = (int64_t)strip * kDecodeStripN;
  // This wave's row group rw and column group cw; its rows row0 .. row0 +
  // Mr - 1 (Mr <= 0: none) and column blocks NCB cw .. of the strip.
  const int rw = wave / WC, cw = wave % WC;
  const int srow0 = slice * SR, row0 = srow0 + rw * WROWS;
  const int Mr = p.M - row0 < WROWS ? p.M - row0 : WROWS;
  const int Ms = p.M - srow0; // rows of the slice (> 0)
  const int8_t *const Ap = p.A + (int64_t)srow0 * p.lda;
  const bool n_edge = n0 + kDecodeStripN > p.N;

  const int total_batches = (p.K + kRowsBatchK - 1) / kRowsBatchK;
  const int b_begin = split * p.batches_per_split;
  int b_end = b_begin + p.batches_per_split;
  if (b_end > total_batches)
    b_end = total_batches;
  const int nb = b_end > b_begin ? b_end - b_begin : 0; // the same for every wave
  const int rot = BT && nb > 0 ? strip % nb : 0; // K-major B: the strip's first batch
  auto batch = [&](int i) { // the split's i-th batch to run (i < nb)
    if constexpr (!BT)
      return b_begin + i;
    const int j = i + rot;
    return b_begin + (j >= nb ? j - nb : j);
  };

  // Loads of the split's batch i into `slot`: this wave's 4 of B's 16 KiB
  // (rows 32 wave .. +31 of the batch) and a quarter of the slice's A rows
  // (rows SR/4 wave ..): A load u of the wave holds slice rows r = SR/4 wave
  // + 8 u .. +7, lane l' fetching chunk (l' % 8) ^ ((r >> 1) & 7) of row
  // r + l'/8 to A_OFF + r * 128 + 16 (l' % 8).
  // No loaded VGPR is live across the loop: with the direct-to-LDS loads
  // pending, the compiler can only wait for a loaded register with vmcnt(0)
  // (it counts the two kinds of load as events that may complete out of
  // order), which would drain the ring at every batch.  For i >= nb every
  // load reads the zero chunk instead, so each step issues the same loads.
  auto issue = [&](int i, uint8_t *slot) {
    const bool live = i < nb;
    const int b = live ? batch(i) : b_begin + i;
    const int64_t k0 = (int64_t)b * kRowsBatchK;
    const bool mask = !live || n_edge || b >= p.k_main_batches;
#pragma unroll
    for (int u = 0; u < Cfg::B_LOADS; ++u) {
      const int q = Cfg::B_LOADS * wave + u; // 1 KiB part q of the batch
      const int row = 8 * q + (lane >> 3), pc = lane & 7;
      const void *src;
      if constexpr (BT) { // storage row n0 + row, chunk pc ^ ((row >> 1) & 7), as A's
        const int c = pc ^ ((row >> 1) & 7);
        const int64_t n = n0 + row, k = k0 + 16 * c;
        src = p.B + n * p.ldb + k;
        if (mask && (!live || n >= p.N || k >= p.K))
          src = tx_zero_chunk;
      } else {
        const int c = pc ^ (row & 7);
        const int64_t k = k0 + row, n = n0 + 16 * c;
        src = p.B + k * p.ldb + n;
        if (mask && (!live || k >= p.K || n >= p.N))
          src = tx_zero_chunk;
      }
      dma16_stream(src, (lds_void *)(slot + q * 1024)); // B is read once per slice
    }
#pragma unroll
    for (int u = 0; u < Cfg::A_LOADS; ++u) {
      const int r = (SR / 4) * wave + 8 * u + (lane >> 3);
      const int c = (lane & 7) ^ ((r >> 1) & 7);
      const int64_t k = k0 + 16 * c;
      const void *src = Ap + (int64_t)r * p.lda + k;
      if (!live || r >= Ms || (b >= p.k_main_batches && k >= p.K))
        src = tx_zero_chunk;
      dma16(src, (lds_void *)(slot + Cfg::A_OFF + (Cfg::A_LOADS * wave + u) * 1024)); // A: re-read by every strip
    }
  };

  // acc[rb][cb]: the 32 x 32 block of rows 32 rb .. of the wave's rows and
  // columns 32 (NCB cw + cb) .. of the strip, as C^T (MFMA A := B columns,
  // MFMA B := A rows): lane l holds row 32 rb + l%32 at columns
  // 32 (NCB cw + cb) + 8 q + 4 (l/32) .. +3 in registers 4 q .. 4 q + 3.
  i32x16_t acc[R32][NCB];
#pragma unroll
  for (int rb = 0; rb < R32; ++rb)
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        acc[rb][cb][r] = 0;

  // MFMAs of one batch from `slot`: four K steps of 32, each R32 x NCB
  // v_mfma_i32_32x32x32_i8.  Lane l's A operand for step ks and row block rb
  // -- slice row WROWS rw + 32 rb + l%32, chunk 2 ks + l/32 -- sits at
  // a_k[ks] + 4 KiB rb (WROWS rw is a multiple of 32: the swizzle is l%32's).
  // K-major B, step ks: storage row 32 NCB cw + l%32 (+4 KiB per block),
  // chunk 2 ks + l/32, swizzled like A's.
  uint32_t tr_off[NCB], a_k[4], bk_k[4];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb)
    tr_off[cb] = tr32_off(lane, NCB * cw + cb);
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const int r = lane & 31;
    const uint32_t ch = 16 * ((2 * ks + (lane >> 5)) ^ ((r >> 1) & 7));
    a_k[ks] = Cfg::A_OFF + (WROWS * rw + r) * 128 + ch;
    bk_k[ks] = (32 * NCB * cw + r) * 128 + ch;
  }
  auto consume = [&](const uint8_t *slot, int i) {
    const uint32_t base = lds_addr(slot);
    const bool tail = BT && batch(i) >= p.k_main_batches;
    auto step = [&](auto ks_c) {
      constexpr int KS = decltype(ks_c)::value;
      i32x4_t a[R32];
      i32x4_t bf[NCB];
      if constexpr (BT) {
        rows_read_k32_kmajor<R32, NCB>(base + bk_k[KS], base + a_k[KS], bf, a);
        if (tail) { // the K tail: B's bytes at or past K
          const int64_t k = (int64_t)batch(i) * kRowsBatchK + 32 * KS + 16 * (lane >> 5);
#pragma unroll
          for (int cb = 0; cb < NCB; ++cb)
            bf[cb] = dec8_mask_k(bf[cb], k, p.K);
        }
      } else {
        v2i_t lo[NCB], hi[NCB];
        rows_read_k32<R32, NCB, KS>(base, tr_off, base + a_k[KS], lo, hi, a);
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb)
          bf[cb] = i32x4_t{lo[cb].x, lo[cb].y, hi[cb].x, hi[cb].y};
      }
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
#pragma unroll
        for (int rb = 0; rb < R32; ++rb)
          acc[rb][cb] = mfma_i8_32(bf[cb], a[rb], acc[rb][cb]);
      }
    };
    step(std::integral_constant<int, 0>());
    step(std::integral_constant<int, 1>());
    step(std::integral_constant<int, 2>());
    step(std::integral_constant<int, 3>());
  };

  // The scales go to LDS by 4-byte direct loads ahead of the first batch, so
  // the first batch's wait covers them: each wave its rows' sa, waves 0 and
  // 1 a half of the strip's sb each.  Rows past M and columns past N read
  // element 0 (their results are not stored).
  if (!p.Ci) { // an int32 C has no scales
    const int m = row0 + lane;
    __builtin_amdgcn_global_load_lds(p.sa + (lane < WROWS && m < p.M ? m : 0),
                                     (lds_void *)(scl + kDecodeStripN + 64 * wave), 4, 0, 0);
    if (wave < 2) {
      const int64_t n = n0 + 64 * wave + lane;
      __builtin_amdgcn_global_load_lds(p.sb + (n < p.N ? n : 0),
                                       (lds_void *)(scl + 64 * wave), 4, 0, 0);
    }
  }
  // Prologue: S - 1 batches in flight; batch i uses slot i % S.
#pragma unroll
  for (int s = 0; s < S - 1; ++s)
    issue(s, ring + s * SLOT);
  // Main loop, unrolled by S so slot addresses are static; the loop is left
  // at the first batch past nb (never skipping a step and going round).  At
  // batch i: wait for this wave's loads of batch i (the S - 2 batches after
  // it stay in flight), barrier (every wave's loads of batch i have landed
  // and every wave has read batch i - 1's slot), issue batch i + S - 1 into
  // that slot, then the MFMAs of batch i.
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

  // C = bf16((float(sum) * sa[m]) * sb[n]): lane l writes row
  // row0 + 32 rb + l%32, columns n0 + 32 cb + 8 q + 4 (l/32) .. +3 (one
  // 8-byte store; single elements where the quad crosses N).
  const int rl = lane & 31, ch = lane >> 5;
  auto epilogue = [&](const i32x16_t (&sum)[R32][NCB]) {
    if (p.Ci) { // int32 C: the sums (C += sum under acc_c), one 16-byte access a quad
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int rb = 0; rb < R32; ++rb) {
            const int m = 32 * rb + rl;
            const i32x4_t v = {sum[rb][cb][4 * q], sum[rb][cb][4 * q + 1],
                               sum[rb][cb][4 * q + 2], sum[rb][cb][4 * q + 3]};
            decode_store_i32(p, row0 + m, m < Mr,
                             n0 + 32 * (NCB * cw + cb) + 8 * q + 4 * ch, v);
          }
      return;
    }
    float sav[R32];
#pragma unroll
    for (int rb = 0; rb < R32; ++rb)
      sav[rb] = scl[kDecodeStripN + 64 * wave + 32 * rb + rl];
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int cs = 32 * (NCB * cw + cb) + 8 * q + 4 * ch; // column in the strip
        const int64_t col = n0 + cs;
        const float4 sb4 = *reinterpret_cast<const float4 *>(scl + cs);
        const float sbv[4] = {sb4.x, sb4.y, sb4.z, sb4.w};
#pragma unroll
        for (int rb = 0; rb < R32; ++rb) {
          const int m = 32 * rb + rl;
          if (m >= Mr || col >= p.N)
            continue;
          float f[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
#pragma clang fp contract(off)
            f[r] = ((float)sum[rb][cb][4 * q + r] * sav[rb]) * sbv[r];
          }
          uint16_t *c = p.C + (int64_t)(row0 + m) * p.ldc + col;
          if (col + 4 <= p.N) {
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
  };
  if (p.ksplit == 1) {
    epilogue(acc);
    return;
  }

  // Publish this split's partial, count arrivals for (slice, strip), and let
  // the last arrival gather: decode_i8.h's protocol and SC1 cache policy
  // (cross-workgroup data moves only through the device-coherent level; every
  // store is acknowledged before the barrier that precedes the counter
  // increment; the last workgroup loads only after its increment returned).
  // A partial block (rb, cb) is 4 KiB: register quad q of every lane at
  // 1 KiB q + 16 l.
  constexpr int kSC1 = 16;
  const int64_t split_bytes = decode_rows_split_bytes(p.slices, strips, SR);
  auto part_rsrc = [&](int q) {
    return __builtin_amdgcn_make_buffer_rsrc(
        reinterpret_cast<uint8_t *>(p.partials) + (int64_t)q * split_bytes, 0, (int)split_bytes,
        0x00020000);
  };
  const int blk0 = ((slice * strips + strip) * kDecodeWaves + wave) * R32 * NCB;
  auto part_off = [&](int rb, int cb, int q) {
    return ((blk0 + NCB * rb + cb) << 12) + (q << 10) + 16 * lane;
  };
  {
    const auto mine = part_rsrc(split);
#pragma unroll
    for (int rb = 0; rb < R32; ++rb)
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const i32x4_t v = {acc[rb][cb][4 * q], acc[rb][cb][4 * q + 1], acc[rb][cb][4 * q + 2],
                             acc[rb][cb][4 * q + 3]};
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4i_t, v), mine,
                                                 part_off(rb, cb, q), 0, kSC1);
        }
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    uint32_t *const ctr = &p.counters[slice * strips + strip];
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
  // Last arrival: add the other splits' partials to its own, 16 or 32 loads
  // per lane in flight per round trip: NQS splits' whole blocks while a wave
  // holds 32 rows; a row block of one split at a time at 64 rows (32 loads
  // there would spill registers).
  constexpr int RBG = R32 == 2 ? 1 : R32;                // row blocks per round trip
  constexpr int NQS = R32 == 2 ? 1 : 32 / (R32 * NCB * 4); // splits per round trip
  for (int q0 = 0; q0 < p.ksplit; q0 += NQS)
#pragma unroll
    for (int rb0 = 0; rb0 < R32; rb0 += RBG) {
      v4i_t v[NQS][RBG][NCB][4];
#pragma unroll
      for (int qq = 0; qq < NQS; ++qq) {
        if (q0 + qq >= p.ksplit || q0 + qq == split)
          continue;
        const auto r = part_rsrc(q0 + qq);
#pragma unroll
        for (int rb = 0; rb < RBG; ++rb)
#pragma unroll
          for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
            for (int q = 0; q < 4; ++q)
              v[qq][rb][cb][q] =
                  __builtin_amdgcn_raw_buffer_load_b128(r, part_off(rb0 + rb, cb, q), 0, kSC1);
      }
#pragma unroll
      for (int qq = 0; qq < NQS; ++qq) {
        if (q0 + qq >= p.ksplit || q0 + qq == split)
          continue;
#pragma unroll
        for (int rb = 0; rb < RBG; ++rb)
#pragma unroll
          for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
              for (int r = 0; r < 4; ++r)
                acc[rb0 + rb][cb][4 * q + r] += v[qq][rb][cb][q][r];
      }
    }
  epilogue(acc);
}

} // namespace txk
