// bf16 / fp16 small-M dot (decode shape) for gfx950:
//   C[m][n] = sum_k A[m][k] * B[k][n]
// with A [M,K] (M <= 96) and B [K,N] row-major, both bf16 or both fp16,
// fp32 accumulation, and C in the operands' type (rounded to nearest even)
// or in fp32 (C = sum, or C += sum for tl.dot's acc).
//
// A dot with a few rows of A reads all of B once and does 2 M FLOPs per
// element of B, so it is HBM-bound; the GEMM tiles would leave most of a
// 64-row tile empty and cover N with a handful of workgroups.  Here a
// workgroup owns a strip of 64 columns (128-byte rows of B), the slice of
// SR = 16 ceil(M / 16) rows and a range of K (split-K), so strips x splits
// workgroups stream B once between them:
//  * B's batches of 128 K rows (16 KiB) go through one LDS ring shared by the
//    4 waves: each wave issues 4 of a batch's 16 direct-to-LDS loads
//    (non-temporal: each byte is read once), waits for its own loads
//    (s_waitcnt vmcnt) and one s_barrier per batch makes the whole batch
//    visible.  The same barrier tells every wave that the slot read one batch
//    earlier is free; the batch S - 1 ahead is loaded into it.
//  * A's rows of the batch (SR x 256 bytes) go into the same slot, a quarter
//    loaded by each wave, each load 4 whole rows; 16-byte chunk c of row r
//    sits at c ^ (r & 15), so the 16 rows one quarter-wave reads with
//    ds_read_b128 fall in 16 bank groups.
//  * B rows are N-contiguous and the MFMA wants K-contiguous elements per
//    column: ds_read_b64_tr_b16 transposes on the LDS read (within a 16-lane
//    group, lane L reads row L / 4, columns 4 (L % 4) .. +3 of a 16-column
//    block; lane i receives column i's 4 K-consecutive elements).  B's
//    16-byte chunk c of row r sits at c ^ (r & 7).
//  * Wave w owns columns 16 w .. 16 w + 15 of the strip for every row of the
//    slice (slices past 64 rows read tiles 4 .. T - 1 in a second block of
//    LDS reads), so every wave has MFMA work at any M:
//    v_mfma_f32_16x16x32_{bf16,f16} with the roles swapped (MFMA A := B
//    columns, MFMA B := A rows), so lane l holds row 16 t + l % 16 at the 4
//    consecutive columns 16 w + 4 (l / 16) .. +3.  No cross-wave reduction:
//    the waves own disjoint outputs.
//  * Split-K: decode_i8.h's exchange (SC1 stores of the fp32 partial, an
//    arrival counter per strip that the last arrival resets; the last
//    arrival gathers).  Partials are kept in lane order, 1 KiB per (wave,
//    row tile).  fp32 addition depends on order, so the last arrival adds
//    the splits' partials in split order 0, 1, .. (its own from registers at
//    its place): the result does not depend on which split arrives last.
//
// K loop in LoopSplit form: batches below k_main_batches load unmasked; the
// rest send B rows >= K, B chunks at or past N and A rows >= M to the
// zero-filled chunk.  An A chunk that crosses K is loaded whole and its
// elements past K are zeroed in registers (they would meet B's zero rows,
// but a row's padding may hold Inf or NaN, and Inf * 0 is NaN).
//
// BT: B stored K-major ([N][K] row-major, row stride ldb; q . k^T with k
// row-major, or a weight kept [out][in]).  A strip is then 64 rows of that
// storage, staged like A's rows (256 bytes of a batch each, chunk c of row r
// at c ^ (r & 15)), and the wave's fragment of columns 16 w .. 16 w + 15 is
// read with ds_read_b128 like an A tile: lane l gets column 16 w + l % 16 at
// K 8 (l / 16) .. +7 of the step, the K indices of the A fragment it meets.
// B's chunk that crosses K is loaded whole too, and zeroed in registers like
// A's.  Each strip starts its split's batches at its own batch (strip mod the
// split's batch count), so its fp32 sums can differ from the row-major form's
// in the last bits.
//
// W = 128: strips of 128 columns, for slices up to 80 rows (three slots of
// 32 KiB of B and the slice's A rows fit the LDS).  Every strip reads all of
// A, so A's re-reads are M / W of B's bytes, and wider strips halve them.
// The batch's B is stored as two 64-column halves in the layout above, and
// wave w owns 16-column blocks 2 w and 2 w + 1 (the second block's B
// fragments read in a block of their own); in K-major B, storage rows
// 32 w .. 32 w + 31.
#pragma once

#include <type_traits>

#include "decode_i8.h"

namespace txk {

typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;

constexpr int kDec16StripN = 64;                                   // columns: 128-byte rows
constexpr int kDec16WideMaxM = 80; // strips of 128 columns: slices up to 80 rows (3 slots)
constexpr int kDec16BatchK = 128;                                  // K rows a batch
constexpr int kDec16MaxM = 96;                                     // one slice of 96 rows
constexpr int64_t kDec16MaxStrips = kDecodeCounterBytes / 4;       // one counter per strip

struct Decode16Args {
  const uint16_t *A;
  const uint16_t *B;
  void *C;
  int32_t c_f32; // C is fp32 (else the operands' 16-bit type)
  int32_t acc_c; // fp32 C: add the sums to C's contents (tl.dot's acc)
  int32_t M, N, K;
  int64_t lda, ldb, ldc; // row strides in elements
  int32_t ksplit;
  int32_t batches_per_split;
  int32_t k_main_batches; // batches with every K row < K (unmasked)
  float *partials;        // [ksplit][strips][4 waves][SR / 16][64 lanes][4] fp32
  uint32_t *counters;     // [strips] arrival counters
};

// Bytes of one split's partials: every strip's SR x W fp32 sums.
__host__ __device__ constexpr int64_t decode16_split_bytes(int64_t strips, int sr,
                                                           int w = kDec16StripN) {
  return strips * sr * w * 4;
}

template <int SR, int W = kDec16StripN> struct Decode16Cfg {
  static_assert(W == 64 || W == 128, "strips of 64 or 128 columns");
  static constexpr int T = SR / 16;                         // 16-row tiles
  static constexpr int JB = W / 64;                         // 16-column blocks a wave
  static constexpr int A_OFF = kDec16BatchK * 2 * W;        // B's batch first
  static constexpr int SLOT = A_OFF + SR * kDec16BatchK * 2; // then SR rows of 256 bytes
  static constexpr int S = 158 * 1024 / SLOT > 8 ? 8 : 158 * 1024 / SLOT;
  static constexpr int B_LOADS = A_OFF / 1024 / kDecodeWaves;                  // 4
  static constexpr int A_LOADS = SR * kDec16BatchK * 2 / 1024 / kDecodeWaves; // SR / 16
  static constexpr int VPB = B_LOADS + A_LOADS;
  static_assert(SR % 16 == 0 && SR >= 16 && SR <= kDec16MaxM, "slices of 16 .. 96 rows");
  static_assert(S >= 3 && (S - 2) * VPB <= 63, "ring depth; vmcnt is 6 bits");
};

// Operands of two K steps (32 rows each, KS and KS + 1) of a batch: the
// wave's B fragments (two transposed reads a step, at `blo` / `bhi` and
// +4 KiB for the second step) and its T A fragments (ds_read_b128 at `a0` /
// `a1`, +4 KiB per 16-row tile), waiting for them before the block ends.
// Outputs are early-clobber: a read lands while later reads of the block
// still use their address registers.
#define TX_D16_TR                                                                           \
  "ds_read_b64_tr_b16 %0, %[blo]\n\tds_read_b64_tr_b16 %1, %[bhi]\n\t"                      \
  "ds_read_b64_tr_b16 %2, %[blo] offset:4096\n\tds_read_b64_tr_b16 %3, %[bhi] offset:4096\n\t"
#define TX_D16_OUT "=&v"(lo[0]), "=&v"(hi[0]), "=&v"(lo[1]), "=&v"(hi[1])
#define TX_D16_IN [blo] "v"(blo), [bhi] "v"(bhi), [a0] "v"(a0), [a1] "v"(a1)
template <int T>
__device__ __forceinline__ void dec16_read_pair(uint32_t blo, uint32_t bhi, uint32_t a0,
                                                uint32_t a1, v2i_t (&lo)[2], v2i_t (&hi)[2],
                                                i32x4_t (&a)[2][T]) {
  if constexpr (T == 1)
    asm volatile(TX_D16_TR "ds_read_b128 %4, %[a0]\n\tds_read_b128 %5, %[a1]\n\t"
                           "s_waitcnt lgkmcnt(0)"
                 : TX_D16_OUT, "=&v"(a[0][0]), "=&v"(a[1][0])
                 : TX_D16_IN
                 : "memory");
  else if constexpr (T == 2)
    asm volatile(TX_D16_TR "ds_read_b128 %4, %[a0]\n\tds_read_b128 %5, %[a0] offset:4096\n\t"
                           "ds_read_b128 %6, %[a1]\n\tds_read_b128 %7, %[a1] offset:4096\n\t"
                           "s_waitcnt lgkmcnt(0)"
                 : TX_D16_OUT, "=&v"(a[0][0]), "=&v"(a[0][1]), "=&v"(a[1][0]), "=&v"(a[1][1])
                 : TX_D16_IN
                 : "memory");
  else if constexpr (T == 3)
    asm volatile(TX_D16_TR "ds_read_b128 %4, %[a0]\n\tds_read_b128 %5, %[a0] offset:4096\n\t"
                           "ds_read_b128 %6, %[a0] offset:8192\n\t"
                           "ds_read_b128 %7, %[a1]\n\tds_read_b128 %8, %[a1] offset:4096\n\t"
                           "ds_read_b128 %9, %[a1] offset:8192\n\t"
                           "s_waitcnt lgkmcnt(0)"
                 : TX_D16_OUT, "=&v"(a[0][0]), "=&v"(a[0][1]), "=&v"(a[0][2]), "=&v"(a[1][0]),
                   "=&v"(a[1][1]), "=&v"(a[1][2])
                 : TX_D16_IN
                 : "memory");
  else
    asm volatile(TX_D16_TR "ds_read_b128 %4, %[a0]\n\tds_read_b128 %5, %[a0] offset:4096\n\t"
                           "ds_read_b128 %6, %[a0] offset:8192\n\t"
                           "ds_read_b128 %7, %[a0] offset:12288\n\t"
                           "ds_read_b128 %8, %[a1]\n\tds_read_b128 %9, %[a1] offset:4096\n\t"
                           "ds_read_b128 %10, %[a1] offset:8192\n\t"
                           "ds_read_b128 %11, %[a1] offset:12288\n\t"
                           "s_waitcnt lgkmcnt(0)"
                 : TX_D16_OUT, "=&v"(a[0][0]), "=&v"(a[0][1]), "=&v"(a[0][2]), "=&v"(a[0][3]),
                   "=&v"(a[1][0]), "=&v"(a[1][1]), "=&v"(a[1][2]), "=&v"(a[1][3])
                 : TX_D16_IN
                 : "memory");
}
#undef TX_D16_IN
#undef TX_D16_OUT
#undef TX_D16_TR

// The same with B K-major: two K steps' B fragments (ds_read_b128 at `b0` /
// `b1`) and the T A fragments of each.
#define TX_D16K_T(t, off)                                                                  \
  "ds_read_b128 %[x0" #t "], %[a0] offset:" #off "\n\tds_read_b128 %[x1" #t "], %[a1] offset:" #off \
  "\n\t"
#define TX_D16K_O(t) [x0##t] "=&v"(a[0][t]), [x1##t] "=&v"(a[1][t])
#define TX_D16K_HEAD "ds_read_b128 %[y0], %[b0]\n\tds_read_b128 %[y1], %[b1]\n\t"
#define TX_D16K_BO [y0] "=&v"(bq[0]), [y1] "=&v"(bq[1])
#define TX_D16K_IN [b0] "v"(b0), [b1] "v"(b1), [a0] "v"(a0), [a1] "v"(a1)
template <int T>
__device__ __forceinline__ void dec16_read_pair_kmajor(uint32_t b0, uint32_t b1, uint32_t a0,
                                                       uint32_t a1, i32x4_t (&bq)[2],
                                                       i32x4_t (&a)[2][T]) {
  if constexpr (T == 1)
    asm volatile(TX_D16K_HEAD TX_D16K_T(0, 0) "s_waitcnt lgkmcnt(0)"
                 : TX_D16K_BO, TX_D16K_O(0)
                 : TX_D16K_IN
                 : "memory");
  else if constexpr (T == 2)
    asm volatile(TX_D16K_HEAD TX_D16K_T(0, 0) TX_D16K_T(1, 4096) "s_waitcnt lgkmcnt(0)"
                 : TX_D16K_BO, TX_D16K_O(0), TX_D16K_O(1)
                 : TX_D16K_IN
                 : "memory");
  else if constexpr (T == 3)
    asm volatile(TX_D16K_HEAD TX_D16K_T(0, 0) TX_D16K_T(1, 4096) TX_D16K_T(2, 8192)
                 "s_waitcnt lgkmcnt(0)"
                 : TX_D16K_BO, TX_D16K_O(0), TX_D16K_O(1), TX_D16K_O(2)
                 : TX_D16K_IN
                 : "memory");
  else
    asm volatile(TX_D16K_HEAD TX_D16K_T(0, 0) TX_D16K_T(1, 4096) TX_D16K_T(2, 8192)
                 TX_D16K_T(3, 12288) "s_waitcnt lgkmcnt(0)"
                 : TX_D16K_BO, TX_D16K_O(0), TX_D16K_O(1), TX_D16K_O(2), TX_D16K_O(3)
                 : TX_D16K_IN
                 : "memory");
}
#undef TX_D16K_IN
#undef TX_D16K_BO
#undef TX_D16K_HEAD
#undef TX_D16K_O
#undef TX_D16K_T

// The A fragments of row tiles 4 .. 4 + N - 1 of two K steps (slices past 64
// rows): ds_read_b128 at a0 / a1 + 16 KiB, +4 KiB per tile.
#define TX_D16M_T(t, off)                                                                  \
  "ds_read_b128 %[p0" #t "], %[a0] offset:" #off "\n\tds_read_b128 %[p1" #t "], %[a1] offset:" #off \
  "\n\t"
#define TX_D16M_O(t) [p0##t] "=&v"(x[0][t]), [p1##t] "=&v"(x[1][t])
#define TX_D16M_IN [a0] "v"(a0), [a1] "v"(a1)
template <int N>
__device__ __forceinline__ void dec16_read_more(uint32_t a0, uint32_t a1, i32x4_t (&x)[2][N]) {
  if constexpr (N == 1)
    asm volatile(TX_D16M_T(0, 16384) "s_waitcnt lgkmcnt(0)" : TX_D16M_O(0) : TX_D16M_IN : "memory");
  else if constexpr (N == 2)
    asm volatile(TX_D16M_T(0, 16384) TX_D16M_T(1, 20480) "s_waitcnt lgkmcnt(0)"
                 : TX_D16M_O(0), TX_D16M_O(1)
                 : TX_D16M_IN
                 : "memory");
  else if constexpr (N == 3)
    asm volatile(TX_D16M_T(0, 16384) TX_D16M_T(1, 20480) TX_D16M_T(2, 24576)
                 "s_waitcnt lgkmcnt(0)"
                 : TX_D16M_O(0), TX_D16M_O(1), TX_D16M_O(2)
                 : TX_D16M_IN
                 : "memory");
  else
    asm volatile(TX_D16M_T(0, 16384) TX_D16M_T(1, 20480) TX_D16M_T(2, 24576)
                 TX_D16M_T(3, 28672) "s_waitcnt lgkmcnt(0)"
                 : TX_D16M_O(0), TX_D16M_O(1), TX_D16M_O(2), TX_D16M_O(3)
                 : TX_D16M_IN
                 : "memory");
}
#undef TX_D16M_IN
#undef TX_D16M_O
#undef TX_D16M_T

template <bool BF>
__device__ __forceinline__ f32x4_t mfma16x16x32(const i32x4_t &a, const i32x4_t &b,
                                                const f32x4_t &c) {
  if constexpr (BF) {
    typedef __bf16 v8_t __attribute__((ext_vector_type(8)));
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8_t, a),
                                                   __builtin_bit_cast(v8_t, b), c, 0, 0, 0);
  } else {
    typedef _Float16 v8_t __attribute__((ext_vector_type(8)));
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8_t, a),
                                                  __builtin_bit_cast(v8_t, b), c, 0, 0, 0);
  }
}

// Zero the 16-bit elements of a fragment at K index `k` .. k + 7 that lie at
// or past K (the chunk that crosses K, in the tail batch).
__device__ __forceinline__ i32x4_t dec16_mask_k(const i32x4_t &v, int64_t k, int64_t K) {
  const int w[4] = {v[0], v[1], v[2], v[3]};
  int o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t lo = k + 2 * i < K ? 0xffffu : 0u;
    const uint32_t hi = k + 2 * i + 1 < K ? 0xffff0000u : 0u;
    o[i] = (int)((uint32_t)w[i] & (lo | hi));
  }
  return i32x4_t{o[0], o[1], o[2], o[3]};
}

// B-only reads of two K steps for a wave's second column block (strips of
// 128 columns): row-major, transposed reads at blo / bhi and +4 KiB;
// K-major, ds_read_b128 at b0 / b1.
__device__ __forceinline__ void dec16_read_b_pair(uint32_t blo, uint32_t bhi, v2i_t (&lo)[2],
                                                  v2i_t (&hi)[2]) {
  asm volatile("ds_read_b64_tr_b16 %0, %[blo]\n\tds_read_b64_tr_b16 %1, %[bhi]\n\t"
               "ds_read_b64_tr_b16 %2, %[blo] offset:4096\n\t"
               "ds_read_b64_tr_b16 %3, %[bhi] offset:4096\n\ts_waitcnt lgkmcnt(0)"
               : "=&v"(lo[0]), "=&v"(hi[0]), "=&v"(lo[1]), "=&v"(hi[1])
               : [blo] "v"(blo), [bhi] "v"(bhi)
               : "memory");
}
__device__ __forceinline__ void dec16_read_bk_pair(uint32_t b0, uint32_t b1, i32x4_t (&bq)[2]) {
  asm volatile("ds_read_b128 %0, %[b0]\n\tds_read_b128 %1, %[b1]\n\ts_waitcnt lgkmcnt(0)"
               : "=&v"(bq[0]), "=&v"(bq[1])
               : [b0] "v"(b0), [b1] "v"(b1)
               : "memory");
}

template <int SR, bool BF, bool BT = false, int W = kDec16StripN>
__global__ void __launch_bounds__(kDecodeWaves * 64, 1) decode16_kernel(Decode16Args p) {
  typedef Decode16Cfg<SR, W> Cfg;
  constexpr int S = Cfg::S, SLOT = Cfg::SLOT, T = Cfg::T, JB = Cfg::JB;
  __shared__ __attribute__((aligned(1024))) uint8_t ring[S * SLOT];
  __shared__ uint32_t last_flag;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = lane >> 4, L = lane & 15;
  // Workgroup -> (strip, split): consecutive workgroups are adjacent strips
  // of one split, so the workgroups running at once read whole stretches of
  // B's rows.
  const int strips = (p.N + W - 1) / W;
  const int strip = blockIdx.x % strips, split = blockIdx.x / strips;
  const int64_t n0 = (int64_t)strip * W;
  const bool n_edge = n0 + W > p.N;

  const int total_batches = (p.K + kDec16BatchK - 1) / kDec16BatchK;
  const int b_begin = split * p.batches_per_split;
  int b_end = b_begin + p.batches_per_split;
  if (b_end > total_batches)
    b_end = total_batches;
  const int nb = b_end > b_begin ? b_end - b_begin : 0; // the same for every wave
  // K-major B: each strip walks its split's batches from its own starting
  // batch (strip mod nb), so the workgroups running at once read rows of B's
  // storage at different K offsets, not all at one offset of rows ldb apart.
  const int rot = BT && nb > 0 ? strip % nb : 0;
  auto batch = [&](int i) { // the split's i-th batch to run (i < nb)
    if constexpr (!BT)
      return b_begin + i;
    const int j = i + rot;
    return b_begin + (j >= nb ? j - nb : j);
  };

  // Loads of the split's batch i into `slot`: B rows 32 wave .. +31 of the
  // batch (load u: rows 8 q .. 8 q + 7, q = 4 wave + u, lane l' fetching
  // chunk (l' % 8) ^ (row & 7) of row 8 q + l' / 8; K-major B: storage rows
  // n0 + 4 q .. +3, lane l' fetching chunk (l' % 16) ^ (row & 15) of row
  // 4 q + l' / 16, as for A) and A rows 4 q .. 4 q + 3 (q = A_LOADS wave + u,
  // lane l' fetching chunk (l' % 16) ^ (row & 15) of row 4 q + l' / 16).  No loaded VGPR is live across the loop (with
  // direct-to-LDS loads pending the compiler could only wait for one with
  // vmcnt(0)).  For i >= nb every load reads the zero chunk, so each step
  // issues the same loads.
  auto issue = [&](int i, uint8_t *slot) {
    const bool live = i < nb;
    const int b = live ? batch(i) : b_begin + i;
    const int64_t k0 = (int64_t)b * kDec16BatchK;
    const bool mask = !live || n_edge || b >= p.k_main_batches;
#pragma unroll
    for (int u = 0; u < Cfg::B_LOADS; ++u) {
      const int q = Cfg::B_LOADS * wave + u;
      const void *src;
      if constexpr (BT) {
        const int r = 4 * q + (lane >> 4);
        const int c = (lane & 15) ^ (r & 15);
        const int64_t n = n0 + r, k = k0 + 8 * c;
        src = p.B + n * p.ldb + k;
        if (mask && (!live || n >= p.N || k >= p.K))
          src = tx_zero_chunk;
      } else {
        // Strips of 128 columns: load q >= 16 fills the second 16 KiB, the
        // batch's columns 64 .. 127 in the same layout.
        const int row = 8 * (q & 15) + (lane >> 3);
        const int c = (lane & 7) ^ (row & 7);
        const int64_t k = k0 + row, n = n0 + 64 * (q >> 4) + 8 * c;
        src = p.B + k * p.ldb + n;
        if (mask && (!live || k >= p.K || n >= p.N))
          src = tx_zero_chunk;
      }
      dma16_stream(src, (lds_void *)(slot + q * 1024)); // B is read once
    }
#pragma unroll
    for (int u = 0; u < Cfg::A_LOADS; ++u) {
      const int q = Cfg::A_LOADS * wave + u;
      const int r = 4 * q + (lane >> 4);
      const int c = (lane & 15) ^ (r & 15);
      const int64_t k = k0 + 8 * c;
      const void *src = p.A + (int64_t)r * p.lda + k;
      if (!live || r >= p.M || (b >= p.k_main_batches && k >= p.K))
        src = tx_zero_chunk;
      dma16(src, (lds_void *)(slot + Cfg::A_OFF + q * 1024)); // A: re-read by every strip
    }
  };

  f32x4_t acc[JB][T]; // [column block][row tile]
#pragma unroll
  for (int jj = 0; jj < JB; ++jj)
#pragma unroll
    for (int t = 0; t < T; ++t)
      acc[jj][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // Per-lane LDS offsets within a slot.  B, K step ks: rows 32 ks + 8 G +
  // L / 4 (lo) and +4 (hi), columns 16 wave + 4 (L % 4) .. +3, i.e. chunk
  // 2 wave + (L % 4) / 2, byte 8 (L % 2); the swizzle takes row & 7, which
  // is L / 4 for lo and L / 4 + 4 for hi in every step, so a step is +4 KiB.
  // A, step ks, tile t: row 16 t + L, chunk (4 ks + G) ^ L: +4 KiB per tile.
  // Column block jj of the wave is block J = JB wave + jj of the strip: in
  // row-major B, the 16 KiB half J / 4 and there block J % 4.
  uint32_t b_lo[JB], b_hi[JB];
#pragma unroll
  for (int jj = 0; jj < JB; ++jj) {
    const int J = JB * wave + jj;
    const int cb = 2 * (J & 3) + ((L & 3) >> 1);
    b_lo[jj] = (J >> 2) * 16384 + (L >> 2) * 128 + ((cb ^ (L >> 2)) << 4) + 8 * (L & 1) +
               8 * G * 128;
    b_hi[jj] = b_lo[jj] + 4 * 128 - ((cb ^ (L >> 2)) << 4) + ((cb ^ ((L >> 2) + 4)) << 4);
  }
  // K-major B, step ks: storage row 16 J + L, chunk (4 ks + G) ^ L.
  uint32_t a_k[4], bk_k[JB][4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    a_k[ks] = Cfg::A_OFF + L * 256 + (((4 * ks + G) ^ L) << 4);
#pragma unroll
    for (int jj = 0; jj < JB; ++jj)
      bk_k[jj][ks] = (16 * (JB * wave + jj) + L) * 256 + (((4 * ks + G) ^ L) << 4);
  }

  auto consume = [&](const uint8_t *slot, int i) {
    const uint32_t base = lds_addr(slot);
    const int b = batch(i);
    const bool tail = b >= p.k_main_batches;
    const int64_t k0 = (int64_t)b * kDec16BatchK;
#pragma unroll
    for (int pr = 0; pr < 2; ++pr) {
      constexpr int T4 = T < 4 ? T : 4; // tiles the first read block brings
      i32x4_t bq[JB][2];
      i32x4_t a4[2][T4];
      if constexpr (BT) {
        dec16_read_pair_kmajor<T4>(base + bk_k[0][2 * pr], base + bk_k[0][2 * pr + 1],
                                   base + a_k[2 * pr], base + a_k[2 * pr + 1], bq[0], a4);
        if constexpr (JB == 2)
          dec16_read_bk_pair(base + bk_k[1][2 * pr], base + bk_k[1][2 * pr + 1], bq[1]);
      } else {
        v2i_t lo[JB][2], hi[JB][2];
        dec16_read_pair<T4>(base + b_lo[0] + pr * 8192, base + b_hi[0] + pr * 8192,
                            base + a_k[2 * pr], base + a_k[2 * pr + 1], lo[0], hi[0], a4);
        if constexpr (JB == 2)
          dec16_read_b_pair(base + b_lo[1] + pr * 8192, base + b_hi[1] + pr * 8192, lo[1],
                            hi[1]);
#pragma unroll
        for (int jj = 0; jj < JB; ++jj)
#pragma unroll
          for (int h = 0; h < 2; ++h)
            bq[jj][h] = i32x4_t{lo[jj][h].x, lo[jj][h].y, hi[jj][h].x, hi[jj][h].y};
      }
      i32x4_t a[2][T];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int t = 0; t < T4; ++t)
          a[h][t] = a4[h][t];
      if constexpr (T > 4) { // slices past 64 rows: tiles 4 .. T - 1
        i32x4_t am[2][T - 4];
        dec16_read_more<T - 4>(base + a_k[2 * pr], base + a_k[2 * pr + 1], am);
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int t = 4; t < T; ++t)
            a[h][t] = am[h][t - 4];
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        i32x4_t bf[JB];
#pragma unroll
        for (int jj = 0; jj < JB; ++jj)
          bf[jj] = bq[jj][h];
        if (tail) {
          const int64_t k = k0 + 32 * (2 * pr + h) + 8 * G;
#pragma unroll
          for (int t = 0; t < T; ++t)
            a[h][t] = dec16_mask_k(a[h][t], k, p.K);
          if constexpr (BT) {
#pragma unroll
            for (int jj = 0; jj < JB; ++jj)
              bf[jj] = dec16_mask_k(bf[jj], k, p.K);
          }
        }
#pragma unroll
        for (int jj = 0; jj < JB; ++jj)
#pragma unroll
          for (int t = 0; t < T; ++t)
            acc[jj][t] = mfma16x16x32<BF>(bf[jj], a[h][t], acc[jj][t]);
      }
    }
  };

  // Prologue: S - 1 batches in flight; batch i uses slot i % S.
#pragma unroll
  for (int s = 0; s < S - 1; ++s)
    issue(s, ring + s * SLOT);
  // Main loop, unrolled by S so slot addresses are static; left at the first
  // batch past nb.  At batch i: wait for this wave's loads of batch i (the
  // S - 2 batches after it stay in flight), barrier (every wave's loads of
  // batch i have landed and every wave has read batch i - 1's slot), issue
  // batch i + S - 1 into that slot, then the MFMAs of batch i.
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

  // C for this lane and column block jj: row 16 t + L, columns
  // n0 + 16 (JB wave + jj) + 4 G .. +3 (one 8-byte store in 16-bit C, 16
  // bytes in fp32; single elements where the quad crosses N).
  auto epilogue = [&](const f32x4_t (&sum)[T], int jj) {
    const int64_t col = n0 + 16 * (JB * wave + jj) + 4 * G;
    if (col >= p.N)
      return;
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const int m = 16 * t + L;
      if (m >= p.M)
        continue;
      const float f[4] = {sum[t][0], sum[t][1], sum[t][2], sum[t][3]};
      if (p.c_f32) {
        float *c = static_cast<float *>(p.C) + (int64_t)m * p.ldc + col;
        if (col + 4 <= p.N) {
          f32x4_t v = sum[t];
          if (p.acc_c)
            v += *reinterpret_cast<const f32x4_t *>(c);
          *reinterpret_cast<f32x4_t *>(c) = v;
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (col + r < p.N)
              c[r] = p.acc_c ? c[r] + f[r] : f[r];
        }
      } else {
        uint16_t *c = static_cast<uint16_t *>(p.C) + (int64_t)m * p.ldc + col;
        if (col + 4 <= p.N) {
          uint2 w;
          w.x = BF ? pk_bf16_rne(f[0], f[1]) : pk_f16_rne(f[0], f[1]);
          w.y = BF ? pk_bf16_rne(f[2], f[3]) : pk_f16_rne(f[2], f[3]);
          *reinterpret_cast<uint2 *>(c) = w;
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (col + r < p.N)
              c[r] = BF ? f32_to_bf16_rne(f[r]) : f32_to_f16_rne(f[r]);
        }
      }
    }
  };
  if (p.ksplit == 1) {
#pragma unroll
    for (int jj = 0; jj < JB; ++jj)
      epilogue(acc[jj], jj);
    return;
  }

  // Publish this split's partial, count arrivals for the strip, and let the
  // last arrival gather: decode_i8.h's protocol and SC1 cache policy (data
  // crosses workgroups only through the device-coherent level; every store
  // is acknowledged before the barrier that precedes the counter increment;
  // the last workgroup loads only after its increment has returned).
  constexpr int kSC1 = 16;
  const int64_t split_bytes = decode16_split_bytes(strips, SR, W);
  auto part_rsrc = [&](int q) {
    return __builtin_amdgcn_make_buffer_rsrc(
        reinterpret_cast<uint8_t *>(p.partials) + (int64_t)q * split_bytes, 0, (int)split_bytes,
        0x00020000);
  };
  // 1 KiB blocks in lane order: column block jj, row tile t at blk0 + jj T + t.
  const int blk0 = (strip * kDecodeWaves + wave) * JB * T;
  {
    const auto mine = part_rsrc(split);
#pragma unroll
    for (int jj = 0; jj < JB; ++jj)
#pragma unroll
      for (int t = 0; t < T; ++t)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4i_t, acc[jj][t]), mine,
                                               ((blk0 + jj * T + t) << 10) + 16 * lane, 0,
                                               kSC1);
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
  // Last arrival: sum = partial 0 + partial 1 + .. in split order, its own
  // from registers; NQ splits' loads in flight before any is used.
  f32x4_t sum[JB][T];
#pragma unroll
  for (int jj = 0; jj < JB; ++jj)
#pragma unroll
    for (int t = 0; t < T; ++t)
      sum[jj][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  constexpr int NQ = 4 / JB;
  for (int q0 = 0; q0 < p.ksplit; q0 += NQ) {
    v4i_t v[NQ][JB][T];
#pragma unroll
    for (int qq = 0; qq < NQ; ++qq)
      if (q0 + qq < p.ksplit && q0 + qq != split) {
        const auto r = part_rsrc(q0 + qq);
#pragma unroll
        for (int jj = 0; jj < JB; ++jj)
#pragma unroll
          for (int t = 0; t < T; ++t)
            v[qq][jj][t] = __builtin_amdgcn_raw_buffer_load_b128(
                r, ((blk0 + jj * T + t) << 10) + 16 * lane, 0, kSC1);
      }
#pragma unroll
    for (int qq = 0; qq < NQ; ++qq)
      if (q0 + qq < p.ksplit)
#pragma unroll
        for (int jj = 0; jj < JB; ++jj)
#pragma unroll
          for (int t = 0; t < T; ++t)
            sum[jj][t] +=
                q0 + qq == split ? acc[jj][t] : __builtin_bit_cast(f32x4_t, v[qq][jj][t]);
  }
#pragma unroll
  for (int jj = 0; jj < JB; ++jj)
    epilogue(sum[jj], jj);
}

} // namespace txk
