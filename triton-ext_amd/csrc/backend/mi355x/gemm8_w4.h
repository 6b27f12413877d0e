// 8-bit operand (int8; fp8 e4m3 / e5m2 in any mix; with MX scales also fp4
// e2m1, two per byte) 256x256x128-byte tile kernel for gfx950, eight waves of
// 128x64 (two per SIMD): C[M,N] = epilogue(A[M,K] . B[K,N]), all row-major.
// A wave's 128 fp32/int32 accumulators stay in arch VGPRs, where the
// per-step block-scale FMA can reach them.
//
// One K step is 128: one scale group of the fp8 block-scaled dot, and one
// v_mfma_f32_16x16x128_f8f6f4 (or two v_mfma_i32_16x16x64_i8) per 16x16 block.
// A lane's operand bytes for a block are K = 32 (l/16) .. +31 (32 bytes,
// the same permutation of K for both operands; int8 splits them into two
// 16-byte halves for its two MFMAs).
//
// Staging (per step, 64 KiB plus the step's scales) is gemm16_w4.h's scheme
// for 8-bit elements: buffer loads into LDS with per-tile lane offsets, the K
// step in the scalar soffset and out-of-range offsets returning zeros (rows
// of A >= M, columns of B >= N, and A's columns >= K in masked steps; B's rows
// >= K lie past the buffer); asm statements, so the compiler keeps no LDS read
// behind them.  LDS stage layout:
//   A [256 rows][128 B], 16-byte chunk c of row r at c ^ ((r >> 1) & 7):
//     the 16 rows one ds_read_b128 touches land in 16 different bank groups;
//   B [128 rows][256 B], chunk c of row k at c ^ (k & 7): the 8 rows one
//     ds_read_b64_tr_b8 touches land in 8 different chunks.
//   sa [256] fp32: sa[m0 + r][kt] (block-scaled only, 4-byte buffer loads);
//   sb [64] fp32: sb[kt][n0/128 + 0..1] (block-scaled only).
// B is N-contiguous; ds_read_b64_tr_b8 hands each lane 8 K-consecutive bytes
// of one column (within a 16-lane group, lane i gets byte i%8 of the words
// read by group lanes 2r + i/8), four reads give the 32 bytes of a block.
//
// Operand roles are swapped (MFMA A := B columns, MFMA B := A rows): the
// MFMA result is C^T and lane l holds C row 16 i + l%16 at the 4 consecutive
// columns 16 j + 4 (l/16) .. +3 of block (i, j).
//
// Block scales: per step, part = A_blk . B_blk (a fresh MFMA), then
// acc = fma(part, sa[m][kb] * sb[kb][n/128], acc).  sb is one value per wave
// (a wave's 128 columns lie in one 128-column block) and sa one per lane and
// row block, so the scale costs one FMA per output element per step.  (The
// reference kernel's order, acc + (part * sa) * sb, rounds three times; this
// rounds twice: the results agree to a few ulp.)
//
// Pipeline: two LDS stages.  A wave holds the 4 B fragments of a step (32
// VGPRs) and streams the A fragments (and scales) one row block ahead.  The
// scale FMAs of a row block run during the next row block, after its own
// MFMAs have had that row block's worth of time to finish.  When the last
// row block's A fragment is in registers every wave is done with the stage:
// one barrier, the loads of step k+2 start going into it (a quarter there,
// the rest spread over row blocks 0..2 of step k+1: a 64 KiB burst would
// stall the load path), and each B fragment is replaced by the next step's
// as soon as the last row block's MFMA has used it.
//
// MX (tl.dot_scaled, EPI_MX_*): e8m0 scales per 32 K elements, applied by
// the MFMA itself (v_mfma_scale_f32_16x16x128_f8f6f4 scale operands, no VALU
// work).  The hardware ties lane l's scale byte to row l%16 of its operand
// and TRUE K group l/16, and a lane's operand bytes are true K 16 (l/16) ..
// +15 and 64 + 16 (l/16) .. +15, so MX reads the fragments in that order
// (A chunks l/16 and 4 + l/16; B rows 16 (l/16) + {0, 8, 64, 72}) instead of
// the unscaled kernels' free permutation.  fp8 (e4m3 / e5m2, formats may
// differ) steps over 128 elements of K; fp4 (e2m1, two per byte) over 256,
// the same 128 bytes, as two MFMAs per block: each takes one 16-byte chunk
// (32 elements, lane l holding true K group l/16 of its 128).
// Scales: per step each scale row holds SG = 4 (fp8) or 8 (fp4) bytes at
// byte offset row * (K/32) + SG kt, which need not be 4-byte aligned: the
// row is staged as NSD dwords from that offset rounded down (4-byte buffer
// loads into LDS), and a lane reads its byte at the row's misalignment
// (row * K/32) % 4 plus its group.  Groups at or past K/32 (only the last
// step can have them) read the next row's bytes and are replaced by 127 in
// that step: their operand data is zero, and only a NaN scale (0xFF) could
// leak into the result.
#pragma once

#include <type_traits>

#include "gemm16_w4.h"

namespace txk {

typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;

// The fp4 form of the scaled MFMA reads 4-dword operands: the intrinsic's
// v4i32 overload, called by its LLVM name (the clang builtin is declared for
// 8-dword operands only).
extern "C" __device__ f32x4_t txk_mfma_scale_16x16x128_f4(i32x4_t, i32x4_t, f32x4_t, int, int,
                                                          int, int, int, int)
    __asm("llvm.amdgcn.mfma.scale.f32.16x16x128.f8f6f4.v4i32.v4i32");

// FA, FB: MFMA format codes of A and B (0 e4m3, 1 e5m2; 4 e2m1 with the MX
// epilogues only); the unscaled fp8 dot takes e4m3 / e5m2 in any mix.
// BT: B is stored K-major ([N][K] row-major, row stride ldb), the layout of
// q . k^T with k row-major or of a weight kept [out][in] (every epilogue but
// MX's; the scales do not depend on B's layout).  Its tile is
// staged exactly like A's ([256 columns][128 K bytes], the same swizzle) and
// read with ds_read_b128: lane l gets column l%16's K bytes 32 (l/16) .. +31,
// the same permutation of K as A's fragment.
template <int OP, int EPI, int FA = 0, int FB = 0, bool BT = false> struct Gemm8W4 {
  static constexpr int BM = 256, BN = 256, BK = 128, NW = 8, WN = 4;
  static constexpr int WTM = 128, WTN = 64, FM = WTM / 16, FN = WTN / 16;
  static constexpr bool SCALED = EPI == EPI_BLOCK128_BF16 || EPI == EPI_BLOCK128_F32;
  static constexpr bool INT = OP == OP_I8;
  static constexpr bool PARTIAL = SCALED; // fresh MFMA per step, VALU scale FMA
  static constexpr bool MX = EPI == EPI_MX_F32 || EPI == EPI_MX_BF16;
  static constexpr bool F4 = MX && FA == 4;
  static constexpr int SG = F4 ? 8 : 4;  // MX: scale groups per K step
  static constexpr int NSD = F4 ? 4 : 2; // MX: dwords staged per scale row
  static constexpr int RS = 4 * NSD;     // MX: LDS bytes per scale row
  static constexpr int A_BYTES = BM * BK, B_BYTES = BK * BN; // 32 KiB each
  static constexpr int SA_OFF = A_BYTES + B_BYTES;
  static constexpr int SB_OFF = SA_OFF + (MX ? BM * RS : BM * 4);
  static constexpr uint32_t STAGE = SB_OFF + (MX ? BN * RS : 256);
  static constexpr int A_DMA = A_BYTES / 1024 / NW, B_DMA = B_BYTES / 1024 / NW; // 4, 4
  static constexpr uint32_t kOOB = 0x80000000u;
  static_assert(OP == OP_I8 || OP == OP_F8, "8-bit operands");
  static_assert(!MX || (OP == OP_F8 && ((FA == 4) == (FB == 4)) && FA >= 0 && FA <= 4 &&
                        FB >= 0 && FB <= 4 && FA != 2 && FA != 3 && FB != 2 && FB != 3),
                "MX operands: e4m3 / e5m2 in any mix, or e2m1 on both sides");
  static_assert(!BT || !MX, "K-major B: not the MX forms");
  static_assert(STAGE % 128 == 0, "stage offsets keep address bits 0-6");
  static_assert(2 * STAGE <= 160 * 1024, "two stages in LDS");

  typedef typename std::conditional<INT, i32x4_t, f32x4_t>::type Acc;

  __device__ __forceinline__ static void buffer_lds4(uint32_t voff, const i32x4_t &rsrc,
                                                     uint32_t soff, uint32_t lds) {
    asm volatile("buffer_load_dword %0, %1, %2 offen lds" ::"v"(voff), "s"(rsrc), "s"(soff),
                 "{m0}"(lds)
                 : "memory");
  }

  // Loads of K step kt into the stage at LDS address st (layout above),
  // issued in four parts: PART 0 = A loads 0, 1 and the scale loads; 1 = A
  // loads 2, 3; 2 = B loads 0, 1; 3 = B loads 2, 3 (each 1 KiB).  Buffer
  // loads with per-lane offsets (see gemm16_w4.h): out-of-range offsets read
  // zeros.  Offsets are recomputed per load rather than kept live through
  // the K loop (registers are the scarce resource of this tile).
  template <bool MASK_MN, bool MASK_K, int PART>
  __device__ __forceinline__ static void issue_part(const GemmArgs &p, int64_t m0, int64_t n0,
                                                    const i32x4_t &ra, const i32x4_t &rb,
                                                    const i32x4_t &rsa, const i32x4_t &rsb,
                                                    int kt, uint32_t st, int wave, bool live) {
    const int lane = threadIdx.x & 63;
    const int k0 = kt * BK;
    typedef Gemm16W4<OP_BF16, EPI_F32, 4> W;
    if (PART < 2) {
#pragma unroll
      for (int i = 2 * PART; i < 2 * PART + 2; ++i) {
        const int j = wave * A_DMA + i;
        const int row = 8 * j + (lane >> 3), pc = lane & 7;
        const int c = pc ^ ((row >> 1) & 7);
        const bool ok = live && (!MASK_MN || m0 + row < p.M) && (!MASK_K || k0 + 16 * c < p.K);
        const uint32_t v = ok ? (uint32_t)(m0 + row) * (uint32_t)p.lda + 16u * c : kOOB;
        W::buffer_lds16(v, ra, (uint32_t)k0, st + j * 1024);
      }
    } else {
#pragma unroll
      for (int i = 2 * (PART - 2); i < 2 * (PART - 2) + 2; ++i) {
        const int j = wave * B_DMA + i;
        if constexpr (BT) { // A's staging: column n0 + row, 16-byte K chunk c
          const int row = 8 * j + (lane >> 3), pc = lane & 7;
          const int c = pc ^ ((row >> 1) & 7);
          const bool ok = live && (!MASK_MN || n0 + row < p.N) && (!MASK_K || k0 + 16 * c < p.K);
          const uint32_t v = ok ? (uint32_t)(n0 + row) * (uint32_t)p.ldb + 16u * c : kOOB;
          W::buffer_lds16(v, rb, (uint32_t)k0, st + A_BYTES + j * 1024);
        } else {
          const int k = 4 * j + (lane >> 4), pc = lane & 15;
          const int c = pc ^ (k & 7);
          const bool ok = live && (!MASK_MN || n0 + 16 * c < p.N);
          const uint32_t v = ok ? (uint32_t)k * (uint32_t)p.ldb + (uint32_t)n0 + 16u * c : kOOB;
          W::buffer_lds16(v, rb, (uint32_t)((int64_t)k0 * p.ldb), st + A_BYTES + j * 1024);
        }
      }
    }
    if constexpr (MX) {
      if (PART == 0 || PART == 2) {
        // scale rows of A (part 0) or B (part 2): lane q of the operand's
        // 256 * NSD dwords stages dword q % NSD of row q / NSD
        const bool isA = PART == 0;
        const int64_t r0 = isA ? m0 : n0, rows = isA ? p.M : p.N;
        const uint32_t dst = st + (isA ? SA_OFF : SB_OFF);
#pragma unroll
        for (int t = 0; t < NSD / 2; ++t) {
          const int q = (wave * (NSD / 2) + t) * 64 + lane;
          const int row = q / NSD, dw = q % NSD;
          const int64_t g = r0 + row;
          const bool ok = live && (!MASK_MN || g < rows);
          const uint32_t v =
              ok ? (((uint32_t)g * (uint32_t)p.sa_ld) & ~3u) + 4u * (uint32_t)dw : kOOB;
          buffer_lds4(v, isA ? rsa : rsb, (uint32_t)(kt * SG),
                      dst + (uint32_t)(wave * (NSD / 2) + t) * 256u);
        }
      }
    }
    if (SCALED && PART == 0) {
      if (wave < 4) {
        const int64_t gm = m0 + 64 * wave + lane;
        const uint32_t v = (live && gm < p.M) ? (uint32_t)gm * (uint32_t)(p.sa_ld * 4) : kOOB;
        buffer_lds4(v, rsa, (uint32_t)kt * 4, st + SA_OFF + wave * 256);
      }
      if (wave == 0) {
        const int64_t nb = (n0 >> 7) + lane;
        const uint32_t v = (live && lane < 2 && nb < p.sb_ld) ? (uint32_t)nb * 4u : kOOB;
        buffer_lds4(v, rsb, (uint32_t)(kt * p.sb_ld * 4), st + SB_OFF);
      }
    }
  }

  // Per-lane LDS addresses (stage 0) of the wave's fragments (wave at row
  // block wm of 128 rows, column block wn of 64 columns), one register each:
  //  * A, row block i: row wm*128 + 16 i + l%16, chunk 2 (l/16) after the
  //    swizzle.  The swizzle term (row >> 1) & 7 = (l%16) >> 1 is the same for
  //    every i, so block i is a + 2048 i; the lane's second chunk is ^ 16.
  //  * B, column block j: row 32 (l/16) + (l%16)/2, chunk 4 wn + j after the
  //    swizzle (c ^ (row & 7)); j only flips chunk bits 0-1, so block j is
  //    b ^ (16 j).  The four transposed reads are +0, +2048, +4096, +6144.
  struct Bases {
    uint32_t a, b;
  };
  __device__ __forceinline__ static void bases(uint32_t lds0, int wm, int wn, Bases &bs) {
    const int lane = threadIdx.x & 63;
    const int G = lane >> 4, L = lane & 15;
    const int row = wm * WTM + L;
    bs.a = lds0 + row * BK + (((MX ? G : 2 * G) ^ ((row >> 1) & 7)) << 4);
    if constexpr (BT) { // like A: column wn*64 + 16 j + l%16, chunk 2 (l/16)
      const int col = wn * WTN + L;
      bs.b = lds0 + A_BYTES + col * BK + (((2 * G) ^ ((col >> 1) & 7)) << 4);
    } else {
      const int k = (MX ? 16 : 32) * G + (L >> 1);
      bs.b = lds0 + A_BYTES + k * BN + (((4 * wn) ^ (k & 7)) << 4) + 8 * (L & 1);
    }
  }

  // MX: per-lane LDS addresses (stage 0) of the scale bytes of A row block 0
  // and B column block 0 (block f is + 16 RS f: 16 f rows further, the same
  // misalignment since 16 f (K/32) % 4 == 0).
  __device__ __forceinline__ static void scale_bases(const GemmArgs &p, int64_t m0, int64_t n0,
                                                     uint32_t lds0, int wm, int wn, uint32_t &xa,
                                                     uint32_t &xb) {
    const int lane = threadIdx.x & 63;
    const int G = lane >> 4, L = lane & 15;
    const uint32_t sld = (uint32_t)p.sa_ld;
    const int ra = wm * WTM + L, cb = wn * WTN + L;
    xa = lds0 + SA_OFF + ra * RS + (((uint32_t)(m0 + ra) * sld) & 3u) + G;
    xb = lds0 + SB_OFF + cb * RS + (((uint32_t)(n0 + cb) * sld) & 3u) + G;
  }

  // MX: the scale operand of block f: byte 0 the lane's group (fp4: byte 1
  // the group of the second MFMA, 4 further).
  __device__ __forceinline__ static int read_sx(uint32_t base, uint32_t so, int f) {
    typedef __attribute__((address_space(3))) uint8_t lds_u8;
    const uint32_t a = base + so + 16 * RS * f;
    int v = *(const lds_u8 *)(uintptr_t)a;
    if constexpr (F4)
      v |= (int)*(const lds_u8 *)(uintptr_t)(a + 4) << 8;
    return v;
  }
  // Scale operand v of step kt with the groups at or past ng set to 127.
  __device__ __forceinline__ static int tail_sx(int v, int kt, int ng) {
    const int G = (threadIdx.x & 63) >> 4;
    if (kt * SG + G >= ng)
      v = (v & ~0xff) | 127;
    if constexpr (F4)
      if (kt * SG + 4 + G >= ng)
        v = (v & 0xff) | (127 << 8);
    return v;
  }

  __device__ __forceinline__ static i32x8_t read_a(const Bases &bs, uint32_t so, int i) {
    typedef __attribute__((address_space(3))) i32x4_t lds_i32x4;
    const uint32_t a0 = bs.a + so + 2048 * i;
    const i32x4_t lo = *(const lds_i32x4 *)(uintptr_t)a0;
    const i32x4_t hi = *(const lds_i32x4 *)(uintptr_t)(a0 ^ (MX ? 64u : 16u));
    i32x8_t r;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      r[t] = lo[t];
      r[4 + t] = hi[t];
    }
    return r;
  }

  __device__ __forceinline__ static i32x8_t read_b(const Bases &bs, uint32_t so, int j) {
    if constexpr (BT) { // column block j: 16 columns further, +2048
      Bases c = bs;
      c.a = bs.b;
      return read_a(c, so, j);
    }
    typedef int v2i __attribute__((ext_vector_type(2)));
    typedef __attribute__((address_space(3))) v2i lds_v2i_t;
    const uint32_t b0 = (bs.b ^ (16u * j)) + so;
    i32x8_t r;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t rows = MX ? (q & 1) * 8 + (q >> 1) * 64 : q * 8;
      const v2i v = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i_t *)(uintptr_t)(b0 + rows * BN));
      r[2 * q] = v.x;
      r[2 * q + 1] = v.y;
    }
    return r;
  }

  __device__ __forceinline__ static Acc mma(const i32x8_t &bcol, const i32x8_t &arow, Acc c) {
    if constexpr (INT) {
      i32x4_t b0, b1, a0, a1;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        b0[t] = bcol[t], b1[t] = bcol[4 + t], a0[t] = arow[t], a1[t] = arow[4 + t];
      }
      c = __builtin_amdgcn_mfma_i32_16x16x64_i8(b0, a0, c, 0, 0, 0);
      return __builtin_amdgcn_mfma_i32_16x16x64_i8(b1, a1, c, 0, 0, 0);
    } else {
      // operand formats FB (MFMA A := B columns) and FA; no hardware scales
      return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bcol, arow, c, FB, FA, 0, 0, 0, 0);
    }
  }

  // MX: acc += (B cols * 2^(sbx - 127)) . (A rows * 2^(sxa - 127)), the
  // scales per 32 K elements as laid out above.
  __device__ __forceinline__ static Acc mma_mx(const i32x8_t &bcol, const i32x8_t &arow, Acc c,
                                               int sbx, int sxa) {
    if constexpr (F4) {
      i32x4_t b0, b1, a0, a1;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        b0[t] = bcol[t], b1[t] = bcol[4 + t], a0[t] = arow[t], a1[t] = arow[4 + t];
      }
      c = txk_mfma_scale_16x16x128_f4(b0, a0, c, 4, 4, 0, sbx, 0, sxa);
      return txk_mfma_scale_16x16x128_f4(b1, a1, c, 4, 4, 1, sbx, 1, sxa);
    } else {
      return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bcol, arow, c, FB, FA, 0, sbx, 0,
                                                               sxa);
    }
  }

  // fp8 K tail (a 16-byte chunk that crosses K is loaded whole; K need not
  // fill whole chunks): zero the bytes of this lane's A fragment at K or
  // beyond in the last step.  Byte t of the fragment is K index
  // kt * BK + 32 (l / 16) + t (chunks 2 (l / 16) and 2 (l / 16) + 1); B's
  // rows past K already read as zeros, and an fp8 NaN code times zero would
  // still be NaN.  (int8 needs nothing: junk times zero is zero.)  A K-major
  // B fragment has the same byte layout and is zeroed alike, for int8 too.
  __device__ __forceinline__ static i32x8_t mask_k(i32x8_t v, int kt, int64_t K) {
    const int64_t rem = K - ((int64_t)kt * BK + 32 * ((threadIdx.x & 63) >> 4));
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      const int64_t vb = rem - 4 * w;
      v[w] &= vb >= 4 ? -1 : vb <= 0 ? 0 : (int)((1u << (8 * vb)) - 1u);
    }
    return v;
  }

  // Ties a value to this point of the program: the compiler otherwise sinks
  // the scale FMAs (pure arithmetic) to the end of the step, where every row
  // block's partial products would be live at once.
  __device__ __forceinline__ static void pin(Acc &v) { asm volatile("" : "+v"(v)); }

  template <bool MASK_MN>
  __device__ __forceinline__ static void run(const GemmArgs &p, int64_t m0, int64_t n0,
                                              uint8_t *smem) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WN, wn = wave % WN;
    TX_PHASE_STAMP(0);
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
    // Ranges end at the 16-byte chunk holding each operand's last element
    // (rows start 16-byte aligned, so that chunk is the row's own).  fp4 A:
    // K and lda count bytes here.
    const i32x4_t ra = make_rsrc(p.A, (uint32_t)((p.M - 1) * p.lda + ((p.K + 15) & ~15ll)));
    const i32x4_t rb = BT ? make_rsrc(p.B, (uint32_t)((p.N - 1) * p.ldb + ((p.K + 15) & ~15ll)))
                          : make_rsrc(p.B, (uint32_t)((p.K - 1) * p.ldb + ((p.N + 15) & ~15ll)));
    i32x4_t rsa = {0, 0, 0, 0}, rsb = {0, 0, 0, 0};
    if (SCALED) {
      rsa = make_rsrc(p.sa, (uint32_t)(p.M * p.sa_ld * 4));
      rsb = make_rsrc(p.sb, (uint32_t)(((p.K + 127) / 128) * p.sb_ld * 4));
    }
    uint32_t xa = 0, xb = 0;
    const int ng = p.sa_ld; // MX: scale groups per row
    if constexpr (MX) {
      // sizes rounded up to whole dwords: every dword read holds at least
      // one byte of the array (its base is 4-byte aligned)
      rsa = make_rsrc(p.sa, (uint32_t)((p.M * p.sa_ld + 3) & ~3ll));
      rsb = make_rsrc(p.sb, (uint32_t)((p.N * p.sa_ld + 3) & ~3ll));
      scale_bases(p, m0, n0, lds0, wm, wn, xa, xb);
    }
    Bases bs;
    bases(lds0, wm, wn, bs);
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
      __builtin_amdgcn_s_waitcnt(0x7 << 4);
      __syncthreads();
    };
    typedef __attribute__((address_space(3))) float lds_f32;
    auto scale = [&](uint32_t so, int i) {
      if constexpr (SCALED) {
        const float sbv = *(const lds_f32 *)(uintptr_t)(lds0 + so + SB_OFF + 4 * (wn >> 1));
        return *(const lds_f32 *)(uintptr_t)(lds0 + so + SA_OFF +
                                             4 * (wm * WTM + 16 * i + (lane & 15))) * sbv;
      } else {
        return 1.f;
      }
    };
    // Pending partial products (fp8) of the previous row block and its scale.
    Acc P[FN];
    float sp = 0.f;
#pragma unroll
    for (int j = 0; j < FN; ++j)
      P[j] = Acc{0, 0, 0, 0};
    auto flush = [&](Acc (&dst)[FN]) {
      if constexpr (PARTIAL) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            dst[j][r] = __builtin_fmaf(P[j][r], sp, dst[j][r]);
          pin(dst[j]);
        }
      }
    };
    if (total > 0) {
      part_of(0, std::integral_constant<int, 0>());
      part_of(0, std::integral_constant<int, 1>());
      part_of(0, std::integral_constant<int, 2>());
      part_of(0, std::integral_constant<int, 3>());
      step_barrier();
      TX_PHASE_STAMP(1);
      part_of(1, std::integral_constant<int, 0>());
      i32x8_t b[FN];
      int sbx[FN]; // MX: B scale operands of the step
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        b[j] = read_b(bs, 0, j);
        sbx[j] = MX ? read_sx(xb, 0, j) : 0;
      }
      // One step from stage so; more: a following step exists (issue its
      // remaining loads in row blocks 0..2, the barrier, refill b from sn);
      // tail: the last step (MX scale groups past K/32 possible).
      auto step = [&](int kt, bool more, auto tail) {
        constexpr bool TAIL = MX && decltype(tail)::value;
        // K-major B's chunk that crosses K is loaded whole too: both operands'
        // bytes past K are zeroed then (int8 included: junk times junk is not 0)
        constexpr bool KTAIL = ((!INT && !MX) || BT) && decltype(tail)::value;
        const uint32_t so = (kt & 1) * STAGE, sn = ((kt + 1) & 1) * STAGE;
        i32x8_t a = read_a(bs, so, 0);
        if constexpr (KTAIL)
          a = mask_k(a, kt, p.K);
        if constexpr (KTAIL && BT) {
#pragma unroll
          for (int j = 0; j < FN; ++j)
            b[j] = mask_k(b[j], kt, p.K);
        }
        float sc = scale(so, 0);
        int sxa = MX ? read_sx(xa, so, 0) : 0;
        if constexpr (TAIL) {
          sxa = tail_sx(sxa, kt, ng);
#pragma unroll
          for (int j = 0; j < FN; ++j)
            sbx[j] = tail_sx(sbx[j], kt, ng);
        }
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          i32x8_t an;
          float sn_;
          int sxn = 0;
          if (i + 1 < FM) {
            an = read_a(bs, so, i + 1);
            if constexpr (KTAIL)
              an = mask_k(an, kt, p.K);
            sn_ = scale(so, i + 1);
            if constexpr (MX)
              sxn = read_sx(xa, so, i + 1);
            if constexpr (TAIL)
              sxn = tail_sx(sxn, kt, ng);
          }
          if (more && i == FM - 1) {
            TX_PHASE_STEP_BARRIER(kt, step_barrier);
            part_of(kt + 2, std::integral_constant<int, 0>());
          }
          Acc Q[FN];
#pragma unroll
          for (int j = 0; j < FN; ++j) {
            if constexpr (PARTIAL) {
              Q[j] = mma(b[j], a, Acc{0, 0, 0, 0});
            } else if constexpr (MX) {
              acc[i][j] = mma_mx(b[j], a, acc[i][j], sbx[j], sxa);
              pin(acc[i][j]);
            } else {
              acc[i][j] = mma(b[j], a, acc[i][j]);
            }
            if (more && i == FM - 1) {
              b[j] = read_b(bs, sn, j);
              if constexpr (MX)
                sbx[j] = read_sx(xb, sn, j);
            }
          }
          if (more && i == 0) part_of(kt + 1, std::integral_constant<int, 1>());
          if (more && i == 1) part_of(kt + 1, std::integral_constant<int, 2>());
          if (more && i == 2) part_of(kt + 1, std::integral_constant<int, 3>());
          // FMAs of the previous row block (the last one of the previous step
          // for i == 0), whose MFMAs have had a row block to finish.
          flush(acc[i == 0 ? FM - 1 : i - 1]);
#pragma unroll
          for (int j = 0; j < FN; ++j)
            P[j] = Q[j];
          sp = sc;
          if (i + 1 < FM) {
            a = an;
            sc = sn_;
            sxa = sxn;
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      };
      for (int kt = 0; kt + 1 < total; ++kt)
        step(kt, true, std::false_type());
      step(total - 1, false, std::true_type());
      flush(acc[FM - 1]);
      __builtin_amdgcn_s_waitcnt(0x7 << 4);
    }
    TX_PHASE_STAMP(2);
    if constexpr (!MASK_MN)
      epilogue_lds(p, m0, n0, wm, wn, acc, lds0);
    else
      epilogue<MASK_MN>(p, m0, n0, wm, wn, acc);
    TX_PHASE_STAMP(3);
    TX_PHASE_DRAIN();
    TX_PHASE_STAMP(4);
  }

  // Epilogue of an interior tile through LDS (the two stages are free once
  // every wave is past the K loop): C is staged row-major and leaves in whole
  // rows, each store instruction writing 1 KiB of contiguous 16-byte chunks
  // (two 512-byte bf16 rows, or one 1 KiB row of 32-bit C per pass of 128
  // rows), rather than the accumulators' own 32-byte pieces of 16 rows.  LDS
  // row r holds 16-byte chunk c at c ^ (r & 31).  The values are final
  // before staging: the row x column scales of the W8A8 epilogue are applied
  // in registers, and accumulation into C happens on the way out.
  __device__ __forceinline__ static void epilogue_lds(const GemmArgs &p, int64_t m0, int64_t n0,
                                                      int wm, int wn, const Acc (&acc)[FM][FN],
                                                      uint32_t lds0) {
    typedef unsigned v2u __attribute__((ext_vector_type(2)));
    typedef unsigned v4u __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) v2u lds_v2u;
    typedef __attribute__((address_space(3))) v4u lds_v4u;
    const int lane = threadIdx.x & 63, t = threadIdx.x;
    constexpr bool W32 = EPI == EPI_I32 || EPI == EPI_F32 || EPI == EPI_BLOCK128_F32 ||
                         EPI == EPI_MX_F32; // 32-bit C
    constexpr int ROWB = W32 ? 1024 : 512, ROWS = W32 ? 128 : 256, CH = ROWB / 16;
    static_assert(ROWS * ROWB <= 2 * STAGE, "staged C fits the two stages");
    static_assert(NW * 64 == 512 && BN == 256 && WTM == 128, "two staging passes split at wm");
    __syncthreads(); // every wave is done reading the stages
#pragma unroll
    for (int pass = 0; pass < (W32 ? 2 : 1); ++pass) {
      if (!W32 || wm == pass) {
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          const int r = (W32 ? 0 : wm * WTM) + 16 * i + (lane & 15);
          float sar = 1.f;
          if (EPI == EPI_ROWCOL_BF16)
            sar = p.sa[m0 + wm * WTM + 16 * i + (lane & 15)];
#pragma unroll
          for (int j = 0; j < FN; ++j) {
            const int col = wn * WTN + 16 * j + 4 * (lane >> 4);
            const Acc &v = acc[i][j];
            if constexpr (W32) {
              const int ch = col >> 2;
              *(lds_v4u *)(uintptr_t)(lds0 + r * ROWB + ((ch ^ (r & 31)) << 4)) =
                  __builtin_bit_cast(v4u, v);
            } else {
              float f[4];
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                if (EPI == EPI_ROWCOL_BF16) {
#pragma clang fp contract(off)
                  f[q] = ((float)v[q] * sar) * p.sb[n0 + col + q];
                } else {
                  f[q] = (float)v[q];
                }
              }
              const int ch = col >> 3;
              *(lds_v2u *)(uintptr_t)(lds0 + r * ROWB + ((ch ^ (r & 31)) << 4) + (col & 7) * 2) =
                  v2u{pk_bf16_rne(f[0], f[1]), pk_bf16_rne(f[2], f[3])};
            }
          }
        }
      }
      __syncthreads();
      const int64_t row0 = m0 + pass * ROWS;
#pragma unroll 4
      for (int q = 0; q < ROWS * CH / 512; ++q) {
        const int idx = q * 512 + t, r = idx / CH, ch = idx % CH;
        const v4u v = *(const lds_v4u *)(uintptr_t)(lds0 + r * ROWB + ((ch ^ (r & 31)) << 4));
        if constexpr (W32) {
          v4u *c = reinterpret_cast<v4u *>(reinterpret_cast<uint32_t *>(p.C) + (row0 + r) * p.ldc +
                                           n0 + ch * 4);
          if (p.accumulate) {
            if constexpr (EPI == EPI_I32) {
              *c = __builtin_bit_cast(v4u, __builtin_bit_cast(i32x4_t, *c) +
                                               __builtin_bit_cast(i32x4_t, v));
            } else {
              *c = __builtin_bit_cast(v4u, __builtin_bit_cast(f32x4_t, *c) +
                                               __builtin_bit_cast(f32x4_t, v));
            }
          } else {
            *c = v;
          }
        } else {
          *reinterpret_cast<v4u *>(reinterpret_cast<uint16_t *>(p.C) + (row0 + r) * p.ldc + n0 +
                                   ch * 8) = v;
        }
      }
      if (W32 && pass == 0)
        __syncthreads(); // the first half is read out before the second is staged
    }
  }

  // Lane l holds, per block (i, j), C[row][col .. col+3] with
  // row = m0 + wm*128 + 16 i + l%16 and col = n0 + wn*64 + 16 j + 4 (l/16).
  template <bool MASK_MN>
  __device__ __forceinline__ static void epilogue(const GemmArgs &p, int64_t m0, int64_t n0,
                                                  int wm, int wn, const Acc (&acc)[FM][FN]) {
    epilogue_t<MASK_MN, FM, FN, WTM, WTN>(p, m0, n0, wm, wn, acc);
  }
  // The same for a wave tile of FM_ x FN_ blocks of 16x16 (WTM_ x WTN_).
  template <bool MASK_MN, int FM_, int FN_, int WTM_, int WTN_>
  __device__ __forceinline__ static void epilogue_t(const GemmArgs &p, int64_t m0, int64_t n0,
                                                    int wm, int wn,
                                                    const Acc (&acc)[FM_][FN_]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < FM_; ++i) {
      const int64_t row = m0 + wm * WTM_ + 16 * i + (lane & 15);
      if (MASK_MN && row >= p.M)
        continue;
      float sar = 1.f;
      if (EPI == EPI_ROWCOL_BF16)
        sar = p.sa[row];
#pragma unroll
      for (int j = 0; j < FN_; ++j) {
        const int64_t col = n0 + wn * WTN_ + 16 * j + 4 * (lane >> 4);
        if (MASK_MN && col >= p.N)
          continue;
        const int64_t off = row * p.ldc + col;
        const Acc &v = acc[i][j];
        if (MASK_MN && col + 4 > p.N) { // the quad crosses N: element by element
          // The quad as scalars: a vector indexed by an element loop that
          // can stop early has compiled to element 0 for every element.
          typedef std::remove_cv_t<std::remove_reference_t<decltype(v[0])>> E;
          const E w[4] = {v[0], v[1], v[2], v[3]};
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            if (col + r >= p.N)
              continue;
            if (EPI == EPI_I32) {
              int32_t *c = reinterpret_cast<int32_t *>(p.C) + off + r;
              *c = p.accumulate ? *c + (int32_t)w[r] : (int32_t)w[r];
            } else if (EPI == EPI_F32 || EPI == EPI_BLOCK128_F32 || EPI == EPI_MX_F32) {
              float *c = reinterpret_cast<float *>(p.C) + off + r;
              *c = p.accumulate ? *c + (float)w[r] : (float)w[r];
            } else {
              float f;
              if (EPI == EPI_ROWCOL_BF16) {
#pragma clang fp contract(off)
                f = ((float)w[r] * sar) * p.sb[col + r];
              } else {
                f = (float)w[r];
              }
              reinterpret_cast<uint16_t *>(p.C)[off + r] = f32_to_bf16_rne(f);
            }
          }
          continue;
        }
        if (EPI == EPI_I32) {
          i32x4_t *c = reinterpret_cast<i32x4_t *>(reinterpret_cast<int32_t *>(p.C) + off);
          *c = p.accumulate ? *c + v : v;
        } else if (EPI == EPI_F32 || EPI == EPI_BLOCK128_F32 || EPI == EPI_MX_F32) {
          f32x4_t *c = reinterpret_cast<f32x4_t *>(reinterpret_cast<float *>(p.C) + off);
          *c = p.accumulate ? *c + v : v;
        } else {
          float f[4];
          if (EPI == EPI_ROWCOL_BF16) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              // (float(acc) * sa[m]) * sb[n], each product rounded (the
              // scale vectors need only 4-byte alignment)
#pragma clang fp contract(off)
              f[r] = ((float)v[r] * sar) * p.sb[col + r];
            }
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r)
              f[r] = (float)v[r];
          }
          uint2 w;
          w.x = pk_bf16_rne(f[0], f[1]);
          w.y = pk_bf16_rne(f[2], f[3]);
          *reinterpret_cast<uint2 *>(reinterpret_cast<uint16_t *>(p.C) + off) = w;
        }
      }
    }
  }
};

template <int OP, int EPI, int FA = 0, int FB = 0, bool BT = false>
__global__ void __launch_bounds__(512, 1) gemm8_w4_kernel(GemmArgs p) {
  typedef Gemm8W4<OP, EPI, FA, FB, BT> G;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * G::STAGE];
  int tm, tn;
  tile_coords(p, tm, tn);
  const GemmArgs q = split_k_args<G::BK, 1, 1, BT, G::SCALED>(p);
  const int64_t m0 = (int64_t)tm * G::BM, n0 = (int64_t)tn * G::BN;
  if (m0 + G::BM <= q.M && n0 + G::BN <= q.N)
    G::template run<false>(q, m0, n0, smem);
  else
    G::template run<true>(q, m0, n0, smem);
}

} // namespace txk
