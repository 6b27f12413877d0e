// int8 W8A8 small-M dot (decode shape) for gfx950:
//   C[m][n] = bf16((float(sum_k A[m][k] * B[k][n]) * sa[m]) * sb[n])
// with A int8 [M,K] (M <= 256), B int8 [K,N] row-major, int32 accumulation;
// or, with no scales, the int32 sums themselves (a plain int8 -> int32
// tt.dot of decode shape: C = sum, or C += sum for tl.dot's acc).
//
// The job is one pass over B, so it is HBM-bound and the kernel is built to
// stream B once with every CU keeping plenty of bytes in flight:
//  * A workgroup owns a strip of 128 columns, a range of K (split-K) and a
//    slice of up to 16 * MT rows (row slices of 64 past M = 64); each of its
//    4 waves takes every 4th batch of 64 K rows (8 KiB of B).
//  * Each wave has a private LDS ring of STAGES slots (4, or 3 past
//    M = 32) fed by global_load_lds_dwordx4 (lane l of a wave-wide load
//    writes 16 bytes at slot + 16 l): 8 loads per batch move 64 rows x 128
//    bytes, 128-byte row segments, straight into LDS with no VGPR staging.
//    MT more loads bring the batch's A fragments into the slot, each lane
//    fetching its own MFMA operand (16 bytes of row-major A) to where it
//    reads it back.  B's loads are non-temporal: each
//    byte is read once, and allocating loads would also have to write back
//    whatever dirty lines they evict (measured: 2.7 vs 5.1 TB/s after a
//    write-heavy kernel).  Waves never synchronise with
//    each other inside the K loop; a wave waits for its own loads only
//    (s_waitcnt vmcnt), STAGES - 1 batches stay in flight behind the one
//    being used.
//  * B rows are N-contiguous but the MFMA wants K-contiguous bytes per
//    column.  ds_read_b64_tr_b8 does the transpose on the LDS read: within a
//    16-lane group, lane i receives byte (i % 8) of the 8-byte words read by
//    group lanes 2r + i/8, r = 0..7.  With group lane L reading row L/2,
//    columns 8(L%2)..+7 of a 16-column block, lane i gets that column's 8
//    K-consecutive bytes; two reads give the 16 bytes a lane holds for
//    v_mfma_i32_16x16x64_i8 (lane l: column l % 16, K 16 (l/16) .. +15).
//  * The 16-byte chunks of each LDS row are XOR-swizzled by row (chunk
//    c ^ (row & 7)) through the choice of global address each lane loads, so
//    the 8 rows one transposed read touches sit in 8 different chunks.
//  * After the K loop the 4 waves' accumulators are summed through LDS.  With
//    split-K each workgroup writes its int32 partial to the workspace and the
//    last workgroup of a column strip (arrival counter) adds the others'
//    partials to its own and applies the epilogue.  Integer addition is
//    exact, so the result does not depend on the order.
//  * Arrival counters: each workgroup of a column strip adds 1; the one that
//    brings the counter to ksplit is the last and sets it back to zero, so a
//    completed launch leaves every counter at zero.  The counters must be
//    zero before the first launch on a workspace.
//
// K loop in LoopSplit form: batches below k_main_batches have every row
// < K and load unmasked; the rest (the peeled tail) send rows >= K, columns
// >= N and rows of A >= M to a zero-filled chunk (tl.load's other=0).
#pragma once

#include "gemm16_dma.h"

namespace txk {

constexpr int kDecodeBatchK = 64;
constexpr int kDecodeStripN = 128;
constexpr int kDecodeWaves = 4;
constexpr uint32_t kMaxSplit = 64;
constexpr int kDecodeMaxM = 256; // 4 row slices of 64
// The workspace starts with a fixed-size counter region (one counter per
// (row slice, column strip), for N up to kDecodeMaxStrips * 128), so the
// counters of one shape never overlap the partials of another that used the
// same workspace before.
constexpr int kDecodeMaxStrips = 4096;
constexpr int64_t kDecodeCounterBytes = (int64_t)(kDecodeMaxM / 64) * kDecodeMaxStrips * 4;

struct DecodeArgs {
  const int8_t *A;
  const int8_t *B;
  uint16_t *C;       // bf16 C of the W8A8 epilogue (when Ci is null)
  int32_t *Ci;       // int32 C of a plain int8 -> int32 dot (no scales), or null
  int32_t acc_c;     // with Ci: add the sums to C's contents (tl.dot's acc)
  const float *sa;
  const float *sb;
  int32_t M, N, K;
  int64_t lda, ldb, ldc;
  int32_t ksplit;            // workgroups per column strip (power of two)
  int32_t slices;            // row slices of 16 * MT rows (M > 16 * MT)
  int32_t batches_per_split;
  int32_t k_main_batches;    // batches with every K row < K (unmasked)
  int32_t *partials;         // [ksplit][M][N rounded up to 4] int32
  uint32_t *counters;        // [slices][ceil(N / 128)] arrival counters
};

typedef int v2i_t __attribute__((ext_vector_type(2)));
typedef int v4i_t __attribute__((ext_vector_type(4))); // the buffer builtins' operand type
typedef __attribute__((address_space(3))) v2i_t lds_v2i;

__device__ __forceinline__ i32x4_t mfma_i8_16(const i32x4_t &a, const i32x4_t &b,
                                              i32x4_t acc) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc, 0, 0, 0);
}

// v_mfma_i32_32x32x32_i8: measured at 4.5 POP/s on the chip (4 waves per CU,
// 4 accumulators each) against 1.6 for v_mfma_i32_16x16x64_i8 (8 per wave),
// so the row decode kernel takes its int8 products 32 x 32 at a time.
__device__ __forceinline__ i32x16_t mfma_i8_32(const i32x4_t &a, const i32x4_t &b,
                                               i32x16_t acc) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, acc, 0, 0, 0);
}

// B operands of the 32x32x32 MFMA in a decode ring slot: a batch of 64 or
// more rows (K) x 128 bytes (columns), 16-byte chunk c of row r
// at c ^ (r & 7).  For K step ks (rows 32 ks .. +31) lane l takes column
// 32 cb + l%32, rows 32 ks + 16 (l/32) .. +15: the 16-lane group g = l/16
// holds columns 16 (g%2) .. +15 of block cb and rows 16 (g/2) .. +15 of the
// step, read as two ds_read_b64_tr_b8 of 8 rows (group lane L reads row
// 16 (g/2) + L/2, +8 for the second, bytes 8 (L%2) .. +7 of chunk
// 2 cb + g%2).  Within a group the 8 rows sit in 8 different chunks.  Each
// further step is 32 rows (4 KiB) on, with the same swizzle.
__device__ __forceinline__ uint32_t tr32_off(int lane, int cb) {
  const int g = lane >> 4, L = lane & 15;
  const int row = 16 * (g >> 1) + (L >> 1);
  return row * 128 + (((2 * cb + (g & 1)) ^ (row & 7)) << 4) + 8 * (L & 1);
}

// s_waitcnt vmcnt(C), the other counters untouched (gfx9 encoding: vmcnt
// bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int C> __device__ __forceinline__ void wait_vmcnt() {
  static_assert(C >= 0 && C <= 63, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((C & 0xf) | ((C >> 4) << 14) | (0x7 << 4) | (0xf << 8));
}

// ds_read_b128 of MT consecutive KiB at `addr` (a lane's 16 bytes each),
// waiting for them in the same asm block: the compiler sees the values
// defined only once they are in the registers.  Outputs are early-clobber
// ("=&v"): a read's data lands while later reads of the block still use
// their address registers, so no output may share a register with an input.
template <int MT>
__device__ __forceinline__ void lds_read_a(uint32_t addr, i32x4_t (&a)[MT]) {
  if constexpr (MT == 1)
    asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=&v"(a[0]) : "v"(addr) : "memory");
  else if constexpr (MT == 2)
    asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %2 offset:1024\n\t"
                 "s_waitcnt lgkmcnt(0)"
                 : "=&v"(a[0]), "=&v"(a[1]) : "v"(addr) : "memory");
  else if constexpr (MT == 3)
    asm volatile("ds_read_b128 %0, %3\n\tds_read_b128 %1, %3 offset:1024\n\t"
                 "ds_read_b128 %2, %3 offset:2048\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(a[0]), "=&v"(a[1]), "=&v"(a[2]) : "v"(addr) : "memory");
  else
    asm volatile("ds_read_b128 %0, %4\n\tds_read_b128 %1, %4 offset:1024\n\t"
                 "ds_read_b128 %2, %4 offset:2048\n\tds_read_b128 %3, %4 offset:3072\n\t"
                 "s_waitcnt lgkmcnt(0)"
                 : "=&v"(a[0]), "=&v"(a[1]), "=&v"(a[2]), "=&v"(a[3]) : "v"(addr) : "memory");
}

// The int32 epilogue of one column quad of row m (columns n .. n + 3, n a
// multiple of 4; row strides are multiples of 4 elements, so the quad is
// 16-byte aligned): C = sum, or C += sum under acc_c; elements past N are
// not touched.
__device__ __forceinline__ void decode_store_i32(const DecodeArgs &p, int64_t m, bool row_in,
                                                 int64_t n, const i32x4_t &sum) {
  if (!row_in || n >= p.N)
    return;
  int32_t *c = p.Ci + m * p.ldc + n;
  if (n + 4 <= p.N) {
    i32x4_t v = sum;
    if (p.acc_c)
      v += *reinterpret_cast<const i32x4_t *>(c);
    *reinterpret_cast<i32x4_t *>(c) = v;
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (n + r < p.N)
        c[r] = p.acc_c ? c[r] + sum[r] : sum[r];
  }
}

// Zero the bytes of a 16-byte fragment at K index k .. k + 15 that lie at or
// past K.
__device__ __forceinline__ i32x4_t dec8_mask_k(const i32x4_t &v, int64_t k, int64_t K) {
  int o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t m = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b)
      m |= (k + 4 * i + b < K ? 0xffu : 0u) << (8 * b);
    o[i] = (int)((uint32_t)v[i] & m);
  }
  return i32x4_t{o[0], o[1], o[2], o[3]};
}

template <int MT> struct DecodeCfg {
  // One slot per wave and ring stage: B's 8 KiB batch, then the wave's A
  // rows of that batch (MT KiB); as many stages as fit 160 KiB (4 for
  // MT <= 2, 3 beyond).
  static constexpr int B_BYTES = kDecodeBatchK * kDecodeStripN; // 8 KiB
  static constexpr int SLOT = B_BYTES + MT * 1024;
  static constexpr int STAGE_BYTES = kDecodeWaves * SLOT;
  static constexpr int STAGES = 160 * 1024 / STAGE_BYTES;
  static constexpr int VM_PER_BATCH = 8 + MT; // B and A loads into LDS per batch
  static_assert(STAGES >= 3, "at least two batches in flight behind the one in use");
  static_assert((STAGES - 1) * VM_PER_BATCH <= 63, "vmcnt is 6 bits");
};

template <int MT>
__global__ void __launch_bounds__(kDecodeWaves * 64, 1)
    decode_i8_kernel(DecodeArgs p) {
  typedef DecodeCfg<MT> Cfg;
  constexpr int STAGES = Cfg::STAGES;
  constexpr int STAGE_BYTES = Cfg::STAGE_BYTES;
  __shared__ __attribute__((aligned(1024))) uint8_t ring[STAGES * STAGE_BYTES];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Workgroup -> (row slice, column strip, K split).  Consecutive pairs are
  // adjacent strips of one split: the workgroups running at once then read
  // whole stretches of B's rows rather than every strip's 128 bytes at a
  // fixed offset of each KiB, which loads some HBM channels far more than
  // others (measured: the strips at offsets 384..511 of each KiB ended
  // 3 us after the rest when a strip's splits were adjacent instead).  With
  // several slices, the slices of one pair go to one XCD (workgroups are
  // dealt to the 8 XCDs round-robin) so they read its B through one L2.
  const int strips = (p.N + kDecodeStripN - 1) / kDecodeStripN;
  const int pairs = strips * p.ksplit;
  int slice = 0, pair = blockIdx.x;
  if (p.slices > 1) {
    if (pairs % 8 == 0) {
      const int j = blockIdx.x / 8;
      slice = j % p.slices;
      pair = 8 * (j / p.slices) + blockIdx.x % 8;
    } else {
      slice = blockIdx.x % p.slices;
      pair = blockIdx.x / p.slices;
    }
  }
  const int strip = pair % strips, split = pair / strips;
  const int64_t n0 = (int64_t)strip * kDecodeStripN;
  // This slice's rows: row0 .. row0 + Mr - 1.
  const int row0 = slice * 16 * MT;
  const int Mr = p.M - row0 < 16 * MT ? p.M - row0 : 16 * MT;
  const int8_t *const Ap = p.A + (int64_t)row0 * p.lda;
  const bool n_edge = n0 + kDecodeStripN > p.N;
  uint8_t *slots[STAGES];
#pragma unroll
  for (int s = 0; s < STAGES; ++s)
    slots[s] = ring + s * STAGE_BYTES + wave * Cfg::SLOT;

  const int total_batches = (p.K + kDecodeBatchK - 1) / kDecodeBatchK;
  const int b_begin = split * p.batches_per_split;
  int b_end = b_begin + p.batches_per_split;
  if (b_end > total_batches)
    b_end = total_batches;
  // This wave's batches: b_begin + wave + 4 i, i < nb.
  const int first = b_begin + wave;
  const int nb = first < b_end ? (b_end - first + kDecodeWaves - 1) / kDecodeWaves : 0;

  // Loads of this wave's batch i (split batch first + 4 i) into `slot`, all
  // direct to LDS: B's 8 KiB, then the A rows, lane l of A load t fetching
  // row 16 t + l%16, K bytes 16 (l/16) .. +15 (its own MFMA operand) to
  // B_BYTES + t KiB + 16 l, where the lane reads it back.  No loaded VGPR
  // is live across the loop: with direct-to-LDS loads pending, the compiler
  // can only wait for a loaded register with vmcnt(0) (it counts the two
  // kinds of load as events that may complete out of order), which drained
  // the ring once a round when A went to registers.  For i >= nb every load
  // reads the zero chunk instead, so each step issues the same loads.
  auto issue = [&](int i, uint8_t *slot) {
    const bool live = i < nb;
    const int b = first + kDecodeWaves * i;
    const int64_t k0 = (int64_t)b * kDecodeBatchK;
    const bool mask = !live || n_edge || b >= p.k_main_batches;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int row = 8 * q + (lane >> 3), pc = lane & 7;
      const int c = pc ^ (row & 7);
      const int64_t k = k0 + row, n = n0 + 16 * c;
      const void *src = p.B + k * p.ldb + n;
      if (mask && (!live || k >= p.K || n >= p.N))
        src = tx_zero_chunk;
      dma16_stream(src, (lds_void *)(slot + q * 1024)); // B is read once
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int m = 16 * t + (lane & 15);
      const int64_t k = k0 + 16 * (lane >> 4);
      const void *src = Ap + (int64_t)m * p.lda + k;
      if (!live || m >= Mr || (b >= p.k_main_batches && k >= p.K))
        src = tx_zero_chunk;
      dma16(src, (lds_void *)(slot + Cfg::B_BYTES + t * 1024)); // A: re-read by other strips
    }
  };

  i32x4_t acc[MT][8];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int j = 0; j < 8; ++j)
      acc[t][j] = i32x4_t{0, 0, 0, 0};

  // MFMAs of one batch from `slot`.  The LDS reads are inline asm blocks
  // that end in s_waitcnt lgkmcnt(0): the compiler cannot see them as reads
  // of memory a direct-to-LDS load may still be filling, so it adds no
  // vmcnt(0) of its own, and the counted waits below keep STAGES - 1 batches
  // in flight.  Each block's outputs are complete when the block ends.
  const int G = lane >> 4, L = lane & 15;
  // Byte offsets (within a slot) of this lane's transposed reads: rows
  // 16 G + L/2 (+8), columns 16 j + 8 (L % 2), chunk j swizzled by row.
  uint32_t tr_off[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int r0 = 16 * G + (L >> 1);
    tr_off[j] = r0 * 128 + ((j ^ (r0 & 7)) << 4) + 8 * (L & 1); // row r0 + 8: +1024
  }
  auto consume = [&](const uint8_t *slot) {
    const uint32_t base = lds_addr(slot);
    i32x4_t a[MT];
    lds_read_a<MT>(base + Cfg::B_BYTES + 16 * lane, a);
    v2i_t lo[8], hi[8];
    // Columns 0..63.
    asm volatile(
        "ds_read_b64_tr_b8 %0, %8\n\tds_read_b64_tr_b8 %1, %8 offset:1024\n\t"
        "ds_read_b64_tr_b8 %2, %9\n\tds_read_b64_tr_b8 %3, %9 offset:1024\n\t"
        "ds_read_b64_tr_b8 %4, %10\n\tds_read_b64_tr_b8 %5, %10 offset:1024\n\t"
        "ds_read_b64_tr_b8 %6, %11\n\tds_read_b64_tr_b8 %7, %11 offset:1024\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(lo[0]), "=&v"(hi[0]), "=&v"(lo[1]), "=&v"(hi[1]), "=&v"(lo[2]), "=&v"(hi[2]),
          "=&v"(lo[3]), "=&v"(hi[3])
        : "v"(base + tr_off[0]), "v"(base + tr_off[1]), "v"(base + tr_off[2]),
          "v"(base + tr_off[3])
        : "memory");
    // Columns 64..127.
    asm volatile(
        "ds_read_b64_tr_b8 %0, %8\n\tds_read_b64_tr_b8 %1, %8 offset:1024\n\t"
        "ds_read_b64_tr_b8 %2, %9\n\tds_read_b64_tr_b8 %3, %9 offset:1024\n\t"
        "ds_read_b64_tr_b8 %4, %10\n\tds_read_b64_tr_b8 %5, %10 offset:1024\n\t"
        "ds_read_b64_tr_b8 %6, %11\n\tds_read_b64_tr_b8 %7, %11 offset:1024\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(lo[4]), "=&v"(hi[4]), "=&v"(lo[5]), "=&v"(hi[5]), "=&v"(lo[6]), "=&v"(hi[6]),
          "=&v"(lo[7]), "=&v"(hi[7])
        : "v"(base + tr_off[4]), "v"(base + tr_off[5]), "v"(base + tr_off[6]),
          "v"(base + tr_off[7])
        : "memory");
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const i32x4_t bf = {lo[j].x, lo[j].y, hi[j].x, hi[j].y};
#pragma unroll
      for (int t = 0; t < MT; ++t)
        acc[t][j] = mfma_i8_16(a[t], bf, acc[t][j]);
    }
  };

  // After the K loop each thread owns a column quad of the strip, columns
  // cq .. cq + 3 with cq = 4 (tid % 32), in the RPT = 2 MT rows tid / 32 + 8 j
  // (j < RPT): four consecutive int32 per row, moved as one 16-byte LDS read
  // and as two 8-byte global accesses.  The epilogue's scales go out first
  // and wait in registers, so the epilogue waits on no memory round trip
  // for them.
  constexpr int RPT = 2 * MT;
  static_assert(RPT * 4 * kDecodeWaves * 64 == MT * 16 * kDecodeStripN, "quads cover the tile");
  const int cq = 4 * (tid & 31), rq = tid >> 5;
  float sbv[4] = {0.f, 0.f, 0.f, 0.f}, sav[RPT];
#pragma unroll
  for (int j = 0; j < RPT; ++j)
    sav[j] = 0.f;
  if (!p.Ci) { // the W8A8 epilogue's scales (an int32 C has none)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      sbv[r] = p.sb[n0 + cq + r < p.N ? n0 + cq + r : 0];
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      const int m = rq + 8 * j;
      sav[j] = p.sa[row0 + (m < Mr ? m : 0)];
    }
  }

  // Prologue: STAGES - 1 batches in flight; batch i uses slot i % STAGES.
#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
    issue(s, slots[s]);
  // Main loop, unrolled by STAGES so slot addresses are static; the loop is
  // left at the first batch past nb (never skipping a step and going round).
  for (int i0 = 0;; i0 += STAGES) {
#pragma unroll
    for (int s = 0; s < STAGES; ++s) {
      const int i = i0 + s;
      if (i >= nb)
        goto k_loop_done;
      // Batch i + STAGES - 1 goes into the slot read at step i - 1: wait for
      // those LDS reads (lgkmcnt 0) before the new loads may overwrite it.
      __builtin_amdgcn_s_waitcnt(0xf | (0x3 << 14) | (0x7 << 4));
      issue(i + STAGES - 1, slots[(s + STAGES - 1) % STAGES]);
      wait_vmcnt<(STAGES - 1) * Cfg::VM_PER_BATCH>(); // batch i landed, later ones need not
      consume(slots[s]);
    }
  }
k_loop_done:
  __builtin_amdgcn_s_waitcnt(0); // every load of the loop has landed
  // Sum the 4 waves' accumulators through LDS (the ring is free now): wave
  // w stores its tile into region w of the ring with plain stores, then every
  // thread adds the 4 copies of its quads.  acc[t][j] register r of lane l:
  // row m = 16 t + 4 (l / 16) + r, column n = 16 j + l % 16; element (m, n)
  // sits at m * 128 + (n ^ (16 * ((m >> 2) & 3))), so the four 16-lane groups
  // of one store hit different banks, and the XOR (bits 4-5 of n) keeps each
  // column quad contiguous.
  constexpr int TILE = MT * 16 * kDecodeStripN; // int32 of the strip's sums
  // wave w's copy at ring + w * TILE * 4 bytes; the flag word after the four
  static_assert(4 * TILE * 4 + 4 <= STAGES * STAGE_BYTES, "reduction tiles exceed the ring");
  int32_t *const red = reinterpret_cast<int32_t *>(ring);
  uint32_t *const flag = reinterpret_cast<uint32_t *>(ring + 4 * TILE * 4);
  auto swz = [](int m, int n) { return m * kDecodeStripN + (n ^ (16 * ((m >> 2) & 3))); };
  __syncthreads();
  {
    int32_t *mine_tile = red + wave * TILE;
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          mine_tile[swz(16 * t + 4 * G + r, 16 * j + L)] = acc[t][j][r];
  }
  __syncthreads();
  i32x4_t wsum[RPT];
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    const int q = swz(rq + 8 * j, cq);
    wsum[j] = *reinterpret_cast<const i32x4_t *>(red + q) +
              *reinterpret_cast<const i32x4_t *>(red + TILE + q) +
              *reinterpret_cast<const i32x4_t *>(red + 2 * TILE + q) +
              *reinterpret_cast<const i32x4_t *>(red + 3 * TILE + q);
  }
  // C = bf16((float(sum) * sa[m]) * sb[n]) for this thread's quads: one
  // 8-byte store per row (ldc and n0 + cq are multiples of 4), single
  // elements where the quad crosses N.  An int32 C takes the sums (plus C's
  // contents under acc_c) as one 16-byte access per row.
  auto epilogue = [&](const i32x4_t (&sum)[RPT]) {
    if (p.Ci) {
#pragma unroll
      for (int j = 0; j < RPT; ++j)
        decode_store_i32(p, row0 + rq + 8 * j, rq + 8 * j < Mr, n0 + cq, sum[j]);
      return;
    }
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      const int m = rq + 8 * j;
      if (m >= Mr)
        continue;
      float f[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
#pragma clang fp contract(off)
        f[r] = ((float)sum[j][r] * sav[j]) * sbv[r];
      }
      uint16_t *c = p.C + (int64_t)(row0 + m) * p.ldc + n0 + cq;
      if (n0 + cq + 4 <= p.N) {
        uint2 w;
        w.x = pk_bf16_rne(f[0], f[1]);
        w.y = pk_bf16_rne(f[2], f[3]);
        *reinterpret_cast<uint2 *>(c) = w;
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (n0 + cq + r < p.N)
            c[r] = f32_to_bf16_rne(f[r]);
      }
    }
  };
  if (p.ksplit == 1) {
    epilogue(wsum);
    return;
  }

  // Publish this split's partial ([split][M][np] int32, np = N rounded up
  // to 4 so that every quad is 16-byte aligned), then count arrivals for the
  // strip.  Cross-workgroup data moves only with the SC1 cache policy (what
  // gfx950 gives agent-scope atomics; here on 16-byte buffer accesses, one
  // per quad): stores write through the XCD's L2 to the device-coherent
  // level and loads read from it, so no fence has to write back or
  // invalidate a whole L2 (an agent-scope release/acquire fence pair costs
  // ~40 us here).  Ordering: every thread's stores are acknowledged
  // (s_waitcnt vmcnt(0): an SC1 store is acknowledged once it has reached
  // that level) before the barrier that precedes the counter increment, and
  // the last workgroup issues its loads only after its increment has
  // returned.
  constexpr int kSC1 = 16; // buffer cache-policy bits: SC1 (gfx940 family)
  const int64_t np = (p.N + 3) & ~3;
  // A split's partial as a buffer resource: offsets stay below M * np * 4
  // bytes (at most 512 MiB for M <= 256, N <= 524288).
  auto part_rsrc = [&](int q) {
    return __builtin_amdgcn_make_buffer_rsrc(p.partials + (int64_t)q * p.M * np, 0,
                                             (int)(p.M * np * 4), 0x00020000);
  };
  const bool quad_in = n0 + cq < p.N;
  {
    const auto mine = part_rsrc(split);
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      const int m = rq + 8 * j;
      if (m < Mr && quad_in)
        __builtin_amdgcn_raw_buffer_store_b128(
            __builtin_bit_cast(v4i_t, wsum[j]), mine,
            (int)(((int64_t)(row0 + m) * np + n0 + cq) * 4), 0, kSC1);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    uint32_t *const ctr = &p.counters[slice * strips + strip];
    const uint32_t old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = old + 1 == (uint32_t)p.ksplit;
    if (last) // every split has arrived: none touches the counter again
      __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *reinterpret_cast<volatile uint32_t *>(flag) = last; // past the reduction tiles
  }
  __syncthreads();
  if (!*reinterpret_cast<volatile uint32_t *>(flag))
    return;
  // Last arrival: add the other splits' partials to its own (still in
  // registers) and apply the epilogue.  The loads are unconditional -- rows
  // past the slice and quads past N read the slice's first quad and are
  // dropped after -- and go out NQ splits at a time before any value is used,
  // so the gather costs one memory round trip per NQ splits.
  i32x4_t sum[RPT];
  int off[RPT]; // byte offset within a split's partial
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    const int m = rq + 8 * j;
    off[j] = (int)((m < Mr && quad_in ? (int64_t)(row0 + m) * np + n0 + cq
                                      : (int64_t)row0 * np + n0) * 4);
    sum[j] = wsum[j];
  }
  constexpr int NQ = 4; // NQ * RPT 16-byte loads in flight per thread (<= 32)
  for (int q0 = 0; q0 < p.ksplit; q0 += NQ) {
    v4i_t v[NQ][RPT];
#pragma unroll
    for (int qq = 0; qq < NQ; ++qq) {
      if (q0 + qq < p.ksplit && q0 + qq != split) {
        const auto r = part_rsrc(q0 + qq);
#pragma unroll
        for (int j = 0; j < RPT; ++j)
          v[qq][j] = __builtin_amdgcn_raw_buffer_load_b128(r, off[j], 0, kSC1);
      }
    }
#pragma unroll
    for (int qq = 0; qq < NQ; ++qq)
      if (q0 + qq < p.ksplit && q0 + qq != split)
#pragma unroll
        for (int j = 0; j < RPT; ++j)
          sum[j] += __builtin_bit_cast(i32x4_t, v[qq][j]);
  }
  epilogue(sum);
}

} // namespace txk
