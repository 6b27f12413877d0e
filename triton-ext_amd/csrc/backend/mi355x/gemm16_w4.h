// bf16/fp16 256x256x64 tile kernel for gfx950: C[M,N] = epilogue(A[M,K] .
// B[K,N]), all row-major: four waves of 128x128.
//
// Why four waves.  The K loop is power-limited, not issue-limited: with
// LDS reads removed the same loop runs at a clock about 15% higher.  A
// 128x128 wave tile (4x4 blocks of 32x32) reuses each A and B fragment four
// times, 512 LDS bytes per MFMA against 768 for 128x64, and its 256 fp32
// accumulators live in AGPRs, one wave per SIMD.
//
// Staging is gemm16_dma.h's layout: direct-to-LDS buffer loads (no VGPR
// staging) into swizzled A [256][64] and B [64][256] tiles, two stages.
// B (N-contiguous) reaches the MFMA through ds_read_b64_tr_b16.
//
// Pipeline: see run().  Each sub-step (16 of K) issues its MFMAs in a fixed
// order with the next sub-step's fragment reads and a share of the staging
// loads between them; one barrier per step frees the stage just read.
//
// Operand roles are swapped (MFMA A := B columns, MFMA B := A rows), so the
// MFMA result is C^T and lane l holds row m = l % 32 of a 32x32 block at
// columns 8 (r/4) + 4 (l/32) + r%4: four consecutive columns per register
// quad, written as one 8-byte (bf16/fp16) or 16-byte (fp32) store.
//
// K loop in LoopSplit form: k_main_steps unmasked steps, then the masked
// ones (zero-filled past K, the tl.load(mask, other=0) of the reference
// kernel); the last step issues only last_ks of its 4 sub-steps.  K and N
// need not fill whole 16-byte chunks: the buffer ranges end at the chunk
// holding an operand's last element, a chunk that crosses K is loaded whole
// and its elements past K are zeroed in registers in the last step (B's rows
// past K already read as zeros), and columns past N only reach accumulators
// the epilogue does not store.
#pragma once

#include "gemm16_dma.h"

// Phase stamps: empty in the library.  A measurement build defines them
// before including this header (bench.py's libtx_ceilings.so) to time a
// tile's phases per wave (gemm8_w4.h takes the same hooks):
//   TX_PHASE_STAMP(i): i = 0 at entry, 1 once step 0 has landed, 2 after the
//     K loop, 3 after the epilogue's stores are issued, 4 after
//     TX_PHASE_DRAIN() (their acknowledgement);
//   TX_PHASE_STEP_BARRIER(kt, barrier): the barrier of main-loop step kt.
#ifndef TX_PHASE_STAMP
#define TX_PHASE_STAMP(i) ((void)0)
#define TX_PHASE_DRAIN() ((void)0)
#define TX_PHASE_STEP_BARRIER(kt, barrier) barrier()
#endif

namespace txk {

typedef short i16x8_t __attribute__((ext_vector_type(8)));

// Raw buffer resource (gfx9 V#): 48-bit base, stride 0, num_records bytes,
// word 3 = 0x00020000 (32-bit data format, no swizzle).  Loads whose offset
// is >= num_records return zeros.  Built from kernel arguments, so uniform.
__device__ __forceinline__ i32x4_t make_rsrc(const void *base, uint32_t bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  i32x4_t r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  r[1] = __builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xffffu));
  r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
  r[3] = 0x00020000;
  return r;
}

// BT: B is stored K-major ([N][K] row-major, row stride ldb), the layout of
// q . k^T with k row-major.  Its tile is staged exactly like A's (rows of 64
// K values, same swizzle) and read with ds_read_b128 instead of transposes.
template <int OP, int EPI, int NW = 4, bool BT = false> struct Gemm16W4 {
  static constexpr int BM = 256, BN = 256, BK = 64;
  // 2x2 waves of 128x128 (NW is the wave count, kept as a parameter for the
  // staging layouts other kernels borrow from this one).
  static_assert(NW == 4, "four waves");
  static constexpr int WM = 2, WN = NW / 2;
  static constexpr int WTM = BM / WM, WTN = BN / WN, FM = WTM / 32, FN = WTN / 32, KS = BK / 16;
  static constexpr int RPS = FM + 2 * FN; // LDS reads per sub-step
  static constexpr int MPS = FM * FN;     // MFMAs per sub-step
  // Staging layouts shared with the DMA tile of the same wave grid.
  typedef Gemm16Dma<OP, BM, BN, BK, WM, WN, 2, EPI> Stage;
  static constexpr int RA = Stage::RA, NCA = Stage::NCA, RBB = Stage::RBB;
  static constexpr int A_BYTES = Stage::A_BYTES, B_BYTES = Stage::B_BYTES;
  static_assert(Stage::NW == NW, "staging partition matches the wave count");
  static_assert(OP == OP_BF16 || OP == OP_F16, "16-bit operands only");

  struct Frags {
    u32x4 a[FM];   // A rows: MFMA B operand
    i16x8_t b[FN]; // B columns (transposed reads): MFMA A operand
  };

  // Fragments of sub-step ks from stage (as, bs).
  __device__ __forceinline__ static void load_frags(const uint8_t *as, const uint8_t *bs, int ks,
                                                    int wm, int wn, Frags &f) {
    const int lane = threadIdx.x & 63;
    const int G = lane >> 4, L = lane & 15;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int row = wm * WTM + i * 32 + (lane & 31);
      const int c = ks * 2 + (lane >> 5);
      f.a[i] = *reinterpret_cast<const u32x4 *>(as + row * RA +
                                                ((c ^ ((row ^ (row >> 3)) & (NCA - 1))) << 4));
    }
#pragma unroll
    for (int j = 0; j < FN; ++j)
      read_b_frag(bs, ks, wn, j, f);
  }

  // B fragment j of sub-step ks: lane l holds column n = l % 32 of block j,
  // K values 8 (l / 32) .. +7 of the sub-step.  Row-major B: two transposed
  // reads; K-major B: one 16-byte read, as for A.
  __device__ __forceinline__ static void read_b_frag(const uint8_t *bs, int ks, int wn, int j,
                                                     Frags &f) {
    const int lane = threadIdx.x & 63;
    if constexpr (BT) {
      const int row = wn * WTN + j * 32 + (lane & 31);
      const int c = ks * 2 + (lane >> 5);
      const u32x4 v = *reinterpret_cast<const u32x4 *>(
          bs + row * RA + ((c ^ ((row ^ (row >> 3)) & (NCA - 1))) << 4));
      f.b[j] = __builtin_bit_cast(i16x8_t, v);
    } else {
      const int G = lane >> 4, L = lane & 15;
      const int n = wn * WTN + j * 32 + 16 * (G & 1) + 4 * (L & 3);
      const int k = ks * 16 + 8 * (G >> 1) + (L >> 2), k4 = k + 4;
      const uint32_t off0 = k * RBB + (((n >> 3) ^ (4 * (k & 3))) << 4) + (n & 7) * 2;
      const uint32_t off1 = k4 * RBB + (((n >> 3) ^ (4 * (k4 & 3))) << 4) + (n & 7) * 2;
      const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_i16x4 *)((__attribute__((address_space(3))) uint8_t *)bs + off0));
      const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_i16x4 *)((__attribute__((address_space(3))) uint8_t *)bs + off1));
      f.b[j] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    }
  }

  // Staging.  Buffer loads into LDS (buffer_load_dwordx4 ... lds): every
  // lane has a fixed 32-bit byte offset per load, computed once per tile, and
  // the K step advances through the scalar soffset, so a step's 16 loads
  // cost no VALU.  Chunks outside the matrix get an offset past the buffer's
  // num_records and the hardware returns zeros -- the tl.load(mask, other=0)
  // of the reference kernel -- with no branch:
  //   * rows of A >= M and columns of B >= N: offset kOOB, fixed per tile;
  //   * rows of B >= K: past the end of B already;
  //   * columns of A >= K (masked steps only): offset kOOB for that step.
  // The loads are asm statements (M0 = LDS destination through an operand
  // constraint), so the compiler's wait-count insertion never holds LDS reads
  // of the other stage behind them; the only wait for them is the vmcnt(0)
  // before the next step barrier.
  static constexpr uint32_t kOOB = 0x80000000u; // > num_records (spans < 2 GiB)

  struct Offsets {
    uint32_t a[Stage::A_DMA]; // A: ((m0 + row) * lda + c * 8) * 2, or kOOB
    uint32_t b[Stage::B_DMA]; // B: (k * ldb + n0 + c * 8) * 2, or kOOB
                              // (BT: ((n0 + row) * ldb + c * 8) * 2)
    int32_t ak[Stage::A_DMA]; // A: K index of the chunk within a step
    int32_t bk[BT ? Stage::B_DMA : 1]; // BT: the same for B
  };

  // Offsets of the loads that staging wave `wave` (0..NW-1) issues.
  template <bool MASK_MN>
  __device__ __forceinline__ static void offsets_q(const GemmArgs &p, int64_t m0, int64_t n0,
                                                   int wave, Offsets &o) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < Stage::A_DMA; ++i) {
      const int j = wave * Stage::A_DMA + i; // 1 KiB block of the A tile
      const int g = j * 64 + lane;           // 16-byte slot in the tile
      const int row = g / NCA, pc = g % NCA;
      const int c = pc ^ ((row ^ (row >> 3)) & (NCA - 1));
      o.ak[i] = c * 8;
      o.a[i] = (MASK_MN && m0 + row >= p.M) ? kOOB : (uint32_t)(((m0 + row) * p.lda + c * 8) * 2);
    }
#pragma unroll
    for (int i = 0; i < Stage::B_DMA; ++i) {
      const int j = wave * Stage::B_DMA + i;
      const int g = j * 64 + lane;
      if constexpr (BT) { // the A scheme over B's N rows
        const int row = g / NCA, pc = g % NCA;
        const int c = pc ^ ((row ^ (row >> 3)) & (NCA - 1));
        o.bk[i] = c * 8;
        o.b[i] = (MASK_MN && n0 + row >= p.N) ? kOOB
                                               : (uint32_t)(((n0 + row) * p.ldb + c * 8) * 2);
      } else {
        const int k = g / Stage::NCB, pc = g % Stage::NCB;
        const int c = pc ^ (4 * (k & 3));
        o.b[i] = (MASK_MN && n0 + c * 8 >= p.N) ? kOOB : (uint32_t)((k * p.ldb + n0 + c * 8) * 2);
      }
    }
  }

  __device__ __forceinline__ static void buffer_lds16(uint32_t voff, const i32x4_t &rsrc,
                                                      uint32_t soff, uint32_t lds) {
    asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(rsrc), "s"(soff),
                 "{m0}"(lds)
                 : "memory");
  }

  // Loads of K step kt into the stage at LDS address st.  MASK_K: test A's
  // columns against K (the tail step).  !live: a step past the end (its
  // stage is never read again): every load reads zeros.
  template <bool MASK_K>
  __device__ __forceinline__ static void issue_q(const GemmArgs &p, const Offsets &o,
                                                 const i32x4_t &ra, const i32x4_t &rb, int kt,
                                                 uint32_t st, int wave, bool live = true) {
    const int k0 = kt * BK;
    const uint32_t sa = (uint32_t)k0 * 2u;
    const uint32_t sb = (uint32_t)((int64_t)k0 * p.ldb * 2);
#pragma unroll
    for (int i = 0; i < Stage::A_DMA; ++i) {
      uint32_t v = o.a[i];
      if (MASK_K && (!live || k0 + o.ak[i] >= p.K))
        v = kOOB;
      buffer_lds16(v, ra, sa, st + (wave * Stage::A_DMA + i) * 1024);
    }
#pragma unroll
    for (int i = 0; i < Stage::B_DMA; ++i) {
      uint32_t v = o.b[i];
      if (MASK_K && !live)
        v = kOOB;
      buffer_lds16(v, rb, sb, st + A_BYTES + (wave * Stage::B_DMA + i) * 1024);
    }
  }

  template <bool MASK_MN>
  __device__ __forceinline__ static void offsets(const GemmArgs &p, int64_t m0, int64_t n0,
                                                 Offsets &o) {
    offsets_q<MASK_MN>(p, m0, n0, __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), o);
  }
  __device__ __forceinline__ static f32x16_t mma(const i16x8_t &bcol, const u32x4 &arow,
                                                 f32x16_t acc) {
    if constexpr (OP == OP_BF16)
      return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, bcol),
                                                     __builtin_bit_cast(bf16x8_t, arow), acc,
                                                     0, 0, 0);
    else
      return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, bcol),
                                                    __builtin_bit_cast(f16x8_t, arow), acc,
                                                    0, 0, 0);
  }

  // Zero the elements at K or beyond in the fragments of sub-step ks of K
  // step kt (the last step): lane l's A fragment (and a K-major B fragment)
  // holds K values 8 c .. 8 c + 7 of the step, c = 2 ks + l / 32.  Row-major
  // B needs nothing: its rows past K lie beyond the buffer and read as zeros.
  __device__ __forceinline__ static void mask_k(Frags &f, int kt, int ks, int64_t K) {
    const int64_t rem = K - ((int64_t)kt * BK + ks * 16 + 8 * ((threadIdx.x & 63) >> 5));
    if (rem >= 8)
      return;
    u32x4 m;
#pragma unroll
    for (int w = 0; w < 4; ++w)
      m[w] = rem >= 2 * w + 2 ? 0xffffffffu : rem == 2 * w + 1 ? 0x0000ffffu : 0u;
#pragma unroll
    for (int i = 0; i < FM; ++i)
      f.a[i] &= m;
    if constexpr (BT) {
#pragma unroll
      for (int j = 0; j < FN; ++j)
        f.b[j] = __builtin_bit_cast(i16x8_t, __builtin_bit_cast(u32x4, f.b[j]) & m);
    }
  }

  __device__ __forceinline__ static void mfmas(const Frags &f, f32x16_t (&acc)[FM][FN]) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
        acc[i][j] = mma(f.b[j], f.a[i], acc[i][j]);
  }

  // One fragment read of sub-step ks: unit u < FM is A fragment u (one
  // ds_read_b128), unit FM + j is B fragment j (two transposed reads).
  __device__ __forceinline__ static void read_unit(const uint8_t *as, const uint8_t *bs, int ks,
                                                   int wm, int wn, int u, Frags &f) {
    const int lane = threadIdx.x & 63;
    const int G = lane >> 4, L = lane & 15;
    if (u < FM) {
      const int row = wm * WTM + u * 32 + (lane & 31);
      const int c = ks * 2 + (lane >> 5);
      f.a[u] = *reinterpret_cast<const u32x4 *>(as + row * RA +
                                                ((c ^ ((row ^ (row >> 3)) & (NCA - 1))) << 4));
    } else {
      read_b_frag(bs, ks, wn, u - FM, f);
    }
  }

  // Staging loads per wave and step, issued in PARTS groups of PER spread
  // over the step (see run()).
  static constexpr int NDMA = Stage::A_DMA + Stage::B_DMA;
  static constexpr int PARTS = 3;
  static constexpr int PER = (NDMA + PARTS - 1) / PARTS;
  static constexpr int NU = FM + FN; // read units per sub-step
  static_assert(NU <= MPS && PER <= MPS, "one read unit and one load per MFMA at most");

  // Load `idx` (0..NDMA-1) of this wave's share of step kt, into stage st.
  template <bool MASK_K>
  __device__ __forceinline__ static void issue_one(const GemmArgs &p, const Offsets &o,
                                                   const i32x4_t &ra, const i32x4_t &rb, int kt,
                                                   uint32_t st, int wave, bool live, int idx) {
    const int k0 = kt * BK;
    if (idx < Stage::A_DMA) {
      uint32_t v = o.a[idx];
      if (MASK_K && (!live || k0 + o.ak[idx] >= p.K))
        v = kOOB;
      buffer_lds16(v, ra, (uint32_t)k0 * 2u, st + (wave * Stage::A_DMA + idx) * 1024);
    } else {
      const int q = idx - Stage::A_DMA;
      uint32_t v = o.b[q];
      if constexpr (BT) {
        if (MASK_K && (!live || k0 + o.bk[q] >= p.K))
          v = kOOB;
        buffer_lds16(v, rb, (uint32_t)k0 * 2u, st + A_BYTES + (wave * Stage::B_DMA + q) * 1024);
      } else {
        if (MASK_K && !live)
          v = kOOB;
        buffer_lds16(v, rb, (uint32_t)((int64_t)k0 * p.ldb * 2),
                     st + A_BYTES + (wave * Stage::B_DMA + q) * 1024);
      }
    }
  }

  // Pipeline (two LDS stages; step kt in stage kt % 2).  A step's 4
  // sub-steps each issue their MFMAs one at a time in a fixed order: after
  // MFMA u (u < NU) read unit u of the next sub-step's fragments; after the
  // last PER MFMAs, one staging load each.  The loads of step kt + 2 are
  // spread over sub-step 3 of step kt and sub-steps 0 (and, four waves, 1)
  // of step kt + 1, rather than issued in one burst: the CU's load path
  // takes a burst of 64 KiB far slower than the MFMAs take to hide it.
  //   sub-step 0: MFMAs ks0, read ks1, loads part 1 of step kt + 1
  //   sub-step 1: MFMAs ks1, read ks2, loads part 2 of step kt + 1 (PARTS 3)
  //   sub-step 2: MFMAs ks2, read ks3
  //   barrier: s_waitcnt vmcnt(0) lgkmcnt(0) (step kt + 1 has landed, every
  //            fragment of step kt is in registers), s_barrier (so for every
  //            wave): stage kt % 2 is free
  //   sub-step 3: MFMAs ks3, read ks0 of step kt + 1, loads part 0 of kt + 2
  template <bool MASK_MN>
  __device__ __forceinline__ static void run(const GemmArgs &p, int64_t m0, int64_t n0,
                                             uint8_t *smem) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WN, wn = wave % WN;
    TX_PHASE_STAMP(0);
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
    constexpr uint32_t STAGE = A_BYTES + B_BYTES;
    auto stage_ptr = [&](int kt) { return smem + (kt & 1) * STAGE; };
    auto stage_addr = [&](int kt) { return lds0 + (kt & 1) * STAGE; };
    // Ranges end at the 16-byte chunk holding each operand's last element
    // (rows start 16-byte aligned, so that chunk is the row's own).
    const int64_t K8 = (p.K + 7) & ~7ll, N8 = (p.N + 7) & ~7ll;
    const i32x4_t ra = make_rsrc(p.A, (uint32_t)(((p.M - 1) * p.lda + K8) * 2));
    const i32x4_t rb = make_rsrc(p.B, BT ? (uint32_t)(((p.N - 1) * p.ldb + K8) * 2)
                                         : (uint32_t)(((p.K - 1) * p.ldb + N8) * 2));
    Offsets o;
    offsets<MASK_MN>(p, m0, n0, o);
    auto step_barrier = [] {
      __builtin_amdgcn_s_waitcnt(0x7 << 4); // vmcnt 0, expcnt 7, lgkmcnt 0
      __syncthreads();
    };
    // Loads [d0, d0 + n) of step kt (masked: the step may lie past K).
    auto issue_range = [&](int kt, int d0, int n, auto mask_k) {
      constexpr bool MASK_K = decltype(mask_k)::value;
#pragma unroll
      for (int d = 0; d < n; ++d)
        if (d0 + d < NDMA)
          issue_one<MASK_K>(p, o, ra, rb, kt, stage_addr(kt), wave, kt < total, d0 + d);
    };
    // One sub-step: the MFMAs of fc; read units of sub-step rks of stage
    // (ras, rbs) into fn (reads); loads [d0, d0 + PER) of step dkt (d0 >= 0).
    auto sub = [&](const Frags &fc, Frags &fn, const uint8_t *ras, int rks, bool reads, int dkt,
                   int d0, auto mask_k) {
      constexpr bool MASK_K = decltype(mask_k)::value;
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int u = i * FN + j;
          acc[i][j] = mma(fc.b[j], fc.a[i], acc[i][j]);
          if (reads && u < NU)
            read_unit(ras, ras + A_BYTES, rks, wm, wn, u, fn);
          const int d = u - (MPS - PER);
          if (d0 >= 0 && d >= 0 && d0 + d < NDMA)
            issue_one<MASK_K>(p, o, ra, rb, dkt, stage_addr(dkt), wave, dkt < total, d0 + d);
          __builtin_amdgcn_sched_barrier(0);
        }
    };

    if (total > 0) {
      issue_range(0, 0, NDMA, std::true_type()); // masked form: K may end in step 0
      step_barrier();
      TX_PHASE_STAMP(1);
      issue_range(1, 0, PER, std::true_type());
      Frags f0, f1;
      load_frags(stage_ptr(0), stage_ptr(0) + A_BYTES, 0, wm, wn, f0);
      // Every step but the last, straight-line.  The first loop's steps
      // load steps kt + 1 and kt + 2 unmasked; the second's masked (the K
      // tail) or dead (past the end).
      auto full_step = [&](int kt, auto mask_k) {
        const uint8_t *as = stage_ptr(kt), *an = stage_ptr(kt + 1);
        sub(f0, f1, as, 1, true, kt + 1, PARTS > 1 ? PER : -1, mask_k);
        sub(f1, f0, as, 2, true, kt + 1, PARTS > 2 ? 2 * PER : -1, mask_k);
        sub(f0, f1, as, 3, true, 0, -1, mask_k);
        TX_PHASE_STEP_BARRIER(kt, step_barrier);
        sub(f1, f0, an, 0, true, kt + 2, 0, mask_k);
      };
      int kt = 0;
      const int unmasked_end = nmain - 2 < total - 1 ? nmain - 2 : total - 1;
      for (; kt < unmasked_end; ++kt)
        full_step(kt, std::false_type());
      for (; kt < total - 1; ++kt)
        full_step(kt, std::true_type());
      // The last step (the peeled K tail when K % BK != 0): only the
      // sub-steps that reach k < K.
      const uint8_t *as = stage_ptr(kt), *bs = as + A_BYTES;
      const int nks = p.last_ks;
      if (nks > 1)
        load_frags(as, bs, 1, wm, wn, f1);
      mask_k(f0, kt, 0, p.K);
      mfmas(f0, acc);
      if (nks > 1) {
        if (nks > 2)
          load_frags(as, bs, 2, wm, wn, f0);
        mask_k(f1, kt, 1, p.K);
        mfmas(f1, acc);
        if (nks > 2) {
          if (nks > 3)
            load_frags(as, bs, 3, wm, wn, f1);
          mask_k(f0, kt, 2, p.K);
          mfmas(f0, acc);
          if (nks > 3) {
            mask_k(f1, kt, 3, p.K);
            mfmas(f1, acc);
          }
        }
      }
      // Loads of a step past the end may still be writing zeros into LDS:
      // let them land before the workgroup can end.
      __builtin_amdgcn_s_waitcnt(0x7 << 4);
    }
    TX_PHASE_STAMP(2);

    epilogue_lds<MASK_MN>(p, m0, n0, wm, wn, acc, lds0);
    TX_PHASE_STAMP(3);
    TX_PHASE_DRAIN();
    TX_PHASE_STAMP(4);
  }

  // Epilogue of a tile through LDS (the two stages, 128 KiB, are free once
  // every wave is past the K loop).  The accumulators' own layout
  // writes 8-byte pieces of 32 rows per store instruction; staged as
  // row-major C in LDS, the tile leaves in whole rows instead: each store
  // instruction writes 1 KiB of contiguous 16-byte chunks, two 512-byte rows
  // of bf16 / fp16 (one pass) or one 1 KiB fp32 row of a half tile (two
  // passes of 128 rows).  Measured: the bf16 epilogue's cycles halved
  // (20.5k -> 10.2k per wave at 4096^3).  LDS row r holds 16-byte chunk c at
  // c ^ (r & 31), so the 32 rows one accumulator store touches, and the two
  // rows one read covers, spread over the banks.  MASK_MN (tiles crossing M
  // or N): rows past M are not stored, nor chunks past N, and the chunk that
  // crosses N is stored element by element.
  template <bool MASK_MN>
  __device__ __forceinline__ static void epilogue_lds(const GemmArgs &p, int64_t m0, int64_t n0,
                                                      int wm, int wn, const f32x16_t (&acc)[FM][FN],
                                                      uint32_t lds0) {
    typedef unsigned v2u __attribute__((ext_vector_type(2)));
    typedef unsigned v4u __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) v2u lds_v2u;
    typedef __attribute__((address_space(3))) v4u lds_v4u;
    const int lane = threadIdx.x & 63, t = threadIdx.x;
    constexpr bool F32 = EPI == EPI_F32;
    constexpr int ROWB = F32 ? 1024 : 512; // LDS bytes per staged row
    constexpr int ROWS = F32 ? 128 : 256;  // rows per pass
    constexpr int CH = ROWB / 16;          // 16-byte chunks per row
    static_assert(ROWS * ROWB <= 2 * (A_BYTES + B_BYTES), "staged C fits the two stages");
    static_assert(NW * 64 == 256 && BN == 256, "one 1 KiB store per wave and pass step");
    __syncthreads(); // every wave is done reading the stages
#pragma unroll
    for (int pass = 0; pass < (F32 ? 2 : 1); ++pass) {
      if (!F32 || wm == pass) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              const int r = (F32 ? 0 : wm * WTM) + i * 32 + (lane & 31);
              const int col = wn * WTN + j * 32 + 8 * g + 4 * (lane >> 5);
              const float v[4] = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                                  acc[i][j][4 * g + 3]};
              if constexpr (F32) {
                const int ch = col >> 2;
                *(lds_v4u *)(uintptr_t)(lds0 + r * ROWB + ((ch ^ (r & 31)) << 4)) =
                    v4u{__builtin_bit_cast(unsigned, v[0]), __builtin_bit_cast(unsigned, v[1]),
                        __builtin_bit_cast(unsigned, v[2]), __builtin_bit_cast(unsigned, v[3])};
              } else {
                const int ch = col >> 3;
                const v2u w = EPI == EPI_BF16 ? v2u{pk_bf16_rne(v[0], v[1]), pk_bf16_rne(v[2], v[3])}
                                              : v2u{pk_f16_rne(v[0], v[1]), pk_f16_rne(v[2], v[3])};
                *(lds_v2u *)(uintptr_t)(lds0 + r * ROWB + ((ch ^ (r & 31)) << 4) + (col & 7) * 2) = w;
              }
            }
      }
      __syncthreads();
      const int64_t row0 = m0 + pass * ROWS;
#pragma unroll 4
      for (int q = 0; q < ROWS * CH / 256; ++q) {
        const int idx = q * 256 + t, r = idx / CH, ch = idx % CH;
        const v4u v = *(const lds_v4u *)(uintptr_t)(lds0 + r * ROWB + ((ch ^ (r & 31)) << 4));
        if constexpr (MASK_MN) {
          constexpr int EPC = F32 ? 4 : 8; // elements per chunk
          const int64_t col = n0 + (int64_t)ch * EPC;
          if (row0 + r >= p.M || col >= p.N)
            continue;
          if (col + EPC > p.N) { // the chunk crosses N
            const int64_t off = (row0 + r) * p.ldc + col;
            // The chunk's words as scalars: indexing the vector by the loop
            // variable compiled to word 0 for every element (measured: fp32
            // C at N = 50 got column 48's value in column 49).
            const unsigned w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int e = 0; e < EPC; ++e) {
              if (col + e < p.N) {
                if constexpr (F32) {
                  float *c = reinterpret_cast<float *>(p.C) + off + e;
                  const float x = __builtin_bit_cast(float, w[e]);
                  *c = p.accumulate ? *c + x : x;
                } else {
                  reinterpret_cast<uint16_t *>(p.C)[off + e] =
                      (uint16_t)(w[e / 2] >> (16 * (e & 1)));
                }
              }
            }
            continue;
          }
        }
        if constexpr (F32) {
          v4u *c = reinterpret_cast<v4u *>(reinterpret_cast<float *>(p.C) + (row0 + r) * p.ldc +
                                           n0 + ch * 4);
          if (p.accumulate) {
            typedef float v4f __attribute__((ext_vector_type(4)));
            *c = __builtin_bit_cast(v4u, __builtin_bit_cast(v4f, *c) + __builtin_bit_cast(v4f, v));
          } else {
            *c = v;
          }
        } else {
          *reinterpret_cast<v4u *>(reinterpret_cast<uint16_t *>(p.C) + (row0 + r) * p.ldc + n0 +
                                   ch * 8) = v;
        }
      }
      if (F32 && pass == 0)
        __syncthreads(); // the first half is read out before the second is staged
    }
  }
};

template <int OP, int EPI, int NW, bool BT = false>
__global__ void __launch_bounds__(NW * 64, 1) gemm16_w4_kernel(GemmArgs p) {
  typedef Gemm16W4<OP, EPI, NW, BT> G;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * (G::A_BYTES + G::B_BYTES)];
  int tm, tn;
  tile_coords(p, tm, tn);
  const GemmArgs q = split_k_args<G::BK, G::BK / 16, 2, BT, false>(p);
  const int64_t m0 = (int64_t)tm * G::BM, n0 = (int64_t)tn * G::BN;
  if (m0 + G::BM <= q.M && n0 + G::BN <= q.N)
    G::template run<false>(q, m0, n0, smem);
  else
    G::template run<true>(q, m0, n0, smem);
}

} // namespace txk
