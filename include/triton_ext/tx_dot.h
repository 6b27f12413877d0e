/*
 * Tiled dot on MI355X (gfx950): plan + launch C-ABI.
 *
 * This is the computation a Triton kernel expresses as
 *
 *     acc = zeros([BM, BN], fp32 | int32)
 *     for k in range(0, K, BK):                 # scf.for over K
 *         a = tl.load(A_blk, mask=k_idx < K, other=0)
 *         b = tl.load(B_blk, mask=k_idx < K, other=0)
 *         acc = tl.dot(a, b, acc)               # tt.dot
 *     tl.store(C_blk, epilogue(acc), mask=...)
 *
 * (tt.dot semantics: triton/language/semantic.py:1480-1571 of triton 3.6.0;
 * the reference's own call sites: R:pass/LoopSplit/06-fused-attention.py:63,85.)
 *
 * The reference has no dot implementation of its own: it ships the plugin
 * registry (TritonExtPassInfra.h) and the LoopSplit pass, and leaves the
 * backend directory empty (R:backend/CMakeLists.txt is 0 bytes).  These entry
 * points are what a backend extension adds behind that registry:
 *   tx_dot_plan_create  runs the registered passes ("arith_intensity",
 *                       "loop_split", "mi355x_dot") over one dot: FLOP/byte
 *                       classification and tile choice, the K-loop split into
 *                       a full-tile main loop and a peeled masked tail
 *                       (R:pass/LoopSplit/LoopSplit.cpp:125-197), and the
 *                       choice of HIP kernel;
 *   tx_dot_launch       enqueues the planned kernels on a HIP stream.
 *
 * All pointers are device pointers (HBM) unless stated; `stream` is a
 * hipStream_t (NULL = the null stream).  Errors are reported by return code;
 * tx_get_last_error() gives the message of the calling thread's last error.
 */
#ifndef TRITON_EXT_AMD_TX_DOT_H
#define TRITON_EXT_AMD_TX_DOT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TX_API __attribute__((visibility("default")))

typedef enum tx_dtype {
  TX_F32 = 0,
  TX_F16 = 1,
  TX_BF16 = 2,
  TX_I8 = 3,
  TX_F8E4M3 = 4, /* OCP e4m3fn (triton fp8e4nv): bias 7, max 448 */
  TX_I32 = 5,
  TX_F8E5M2 = 6, /* OCP e5m2 (triton fp8e5): bias 15, inf and NaN codes */
  /* OCP e2m1 (fp4), two per byte along K, element k in the low nibble of
   * its byte when k is even (tl.dot_scaled with lhs_k_pack / rhs_k_pack):
   * A is [M][K/2] bytes, B is [K/2][N] bytes.  Row strides stay in
   * elements: lda counts K elements (bytes = lda / 2), ldb counts N
   * elements of a packed row (bytes = ldb). */
  TX_F4E2M1 = 7,
} tx_dtype;

typedef enum tx_scale_mode {
  TX_SCALE_NONE = 0,
  /* W8A8: C[m][n] = bf16((float(acc_i32[m][n]) * sa[m]) * sb[n]) */
  TX_SCALE_ROWCOL = 1,
  /* fp8 block scales: for each 128-wide K block kb,
   *   acc[m][n] += dot_f32(Aq[m][kb], Bq[kb][n]) * sa[m][kb] * sb[kb][n/128]
   * sa is [M][ceil(K/128)], sb is [ceil(K/128)][ceil(N/128)], row-major. */
  TX_SCALE_BLOCK128 = 2,
  /* tl.dot_scaled microscaling (OCP MX): e8m0 scales, one per 32 K elements
   * of each operand row (A) or column (B):
   *   C[m][n] = sum_k (A[m][k] * 2^(sa[m][k/32] - 127)) *
   *                   (B[k][n] * 2^(sb[n][k/32] - 127))
   * sa is uint8 [M][K/32] and sb uint8 [N][K/32] (B's scales indexed by
   * column first, as tl.dot_scaled's rhs_scale; not transposed), both
   * row-major and packed, 4-byte aligned.  Scale 0xFF is NaN.  Operands
   * e4m3 / e5m2 (either mix) or e2m1 on both sides; K % 32 == 0; C fp32 or
   * bf16 (round to nearest even).
   * One operand may instead be TX_BF16 with no scale (its scale pointer is
   * not read): the MX operand is upcast to bf16, bf16(x * 2^(s - 127)) to
   * nearest even, and a bf16 dot with fp32 accumulation runs on it, as
   * tl.dot_scaled specifies (T:language/core.py:2072-2076).  The upcast goes
   * to the workspace (plan->workspace_bytes: the MX operand at 2 bytes per
   * element). */
  TX_SCALE_MX32 = 3,
  /* tl.dot_scaled with e4m3 scales, one per 16 K elements (the scale size
   * Triton takes for fp8e4nv scale tensors, T:language/semantic.py:1597-1609;
   * NVFP4): e2m1 operands, sa uint8 e4m3 [M][K/16], sb [N][K/16], 4-byte
   * aligned; one side may be TX_BF16 with no scale.  gfx950's scaled MFMA
   * takes e8m0 scales only, so each e2m1 operand is upcast to bf16
   * (x * decoded scale: exact in bf16) into the workspace and the bf16 tile
   * runs; K % 16 == 0; C fp32 or bf16. */
  TX_SCALE_NV16 = 4,
} tx_scale_mode;

typedef enum tx_bound {
  TX_BOUND_UNKNOWN = 0,
  TX_BOUND_MFMA = 1, /* arithmetic intensity above the ridge point */
  TX_BOUND_HBM = 2,  /* below the ridge point */
} tx_bound;

typedef enum tx_status {
  TX_OK = 0,
  TX_ERR_INVALID = 1,     /* bad descriptor, NULL pointer, misaligned stride */
  TX_ERR_UNSUPPORTED = 2, /* valid dot that no kernel here implements */
  TX_ERR_HIP = 3,         /* a HIP runtime call failed */
  TX_ERR_NO_DEVICE = 4,   /* no gfx950 device visible */
  TX_ERR_WORKSPACE = 5,   /* workspace missing or too small */
  TX_ERR_NO_PASS = 6,     /* a required extension pass is not registered */
} tx_status;

typedef enum tx_kernel {
  TX_KERNEL_NONE = 0,
  TX_KERNEL_GEMM_16BIT = 1, /* bf16/fp16 tile, MFMA 32x32x16, LDS-staged          */
  TX_KERNEL_GEMM_I8 = 2,    /* int8 tile, MFMA 16x16x64 (32x32x32 small tiles)   */
  TX_KERNEL_DECODE_I8 = 3,  /* int8 W8A8 decode shapes, MFMA 16x16x64 (M <= 48)
                             * or 32x32x32 (row slices, M <= 1024; these also
                             * with B K-major)                                */
  TX_KERNEL_GEMM_F8 = 4,    /* fp8 e4m3 tile, MFMA 16x16x128 (32x32x64 small)    */
  TX_KERNEL_GEMM_MX = 5,    /* MX fp8 / fp4 tile, scaled MFMA 16x16x128 (e8m0)   */
  TX_KERNEL_GEMM_MX_BF16 = 6, /* MX x bf16: MX operand upcast to bf16 in the
                               * workspace, then the bf16 tile              */
  TX_KERNEL_DECODE_16BIT = 7, /* bf16/fp16 decode shapes (M <= 96, no scales):
                               * B streamed once, MFMA 16x16x32              */
  TX_KERNEL_DECODE_F8 = 8,    /* 8-bit decode shapes (M <= 64): fp8 unscaled or
                               * with 128-block scales, and int8 (int32 C or
                               * W8A8, M <= 48) with B K-major; B streamed
                               * once, MFMA 16x16x128 (int8: 16x16x64)       */
} tx_kernel;

/* Bit flags for tx_dot_desc.flags */
#define TX_FLAG_NO_LOOP_SPLIT 0x1 /* run every K step masked (no peeling) */
/* B is stored K-major: [N][K] row-major with row stride ldb (0 = K), the
 * layout of tl.dot(q, tl.trans(k)) / q @ k.T with k row-major, and of a
 * weight kept [out][in].  Supported for bf16/fp16 operands on the 256x256x64
 * tile and the 16-bit decode kernel, and for every 8-bit dot but MX (int8 ->
 * int32, W8A8, unscaled and block-scaled fp8) on the 256x256x128 tile, the
 * 8-bit decode kernel (M <= 64; int8 M <= 48) and, for int8, the row decode
 * kernel (its 64 / 128 / 256-row slices). */
#define TX_FLAG_B_KMAJOR 0x2
/* C = C + A . B: the accumulator operand of tl.dot(a, b, acc) and
 * tl.dot_scaled(..., acc) (R:pass/LoopSplit/06-fused-attention.py:85).  C
 * must be TX_F32 or TX_I32; the kernel adds its finished fp32 / int32 sum to
 * C's contents (int32 exactly; fp32 in one more rounding than an MFMA chain
 * seeded with C).  Not for the W8A8 decode path (bf16 C). */
#define TX_FLAG_ACCUMULATE 0x4

typedef struct tx_dot_desc {
  int64_t M, N, K;
  /* Row strides in elements of A [M,K], B [K,N], C [M,N] (all row-major;
   * B [N][K] with TX_FLAG_B_KMAJOR); 0 means packed (K, N or K, N).  Row
   * strides in bytes must be multiples of 16.  The kernels load 16-byte
   * chunks: a row's last chunk is read whole, up to 15 bytes past its last
   * element (never past that element's 4 KiB page, since rows and chunks
   * start 16-byte aligned); the bytes past K or N do not reach the result. */
  int64_t lda, ldb, ldc;
  int32_t a_type, b_type, c_type; /* tx_dtype */
  int32_t scale_mode;             /* tx_scale_mode */
  /* Tile sizes; 0 lets the arith_intensity pass choose. */
  int32_t block_m, block_n, block_k;
  int32_t flags;
} tx_dot_desc;

struct tx_dot_plan {
  tx_dot_desc desc; /* resolved copy (strides and tiles filled in) */

  /* arith_intensity pass: algorithmic work (each operand read once, C
   * written once, scales read once) and the roofline it implies. */
  double flops, bytes, intensity; /* FLOP, bytes, FLOP/byte */
  double peak_flops, peak_bw;     /* MI355X peaks for this dtype, per s */
  double ridge;                   /* peak_flops / peak_bw */
  double roofline_us;             /* max(flops/peak, bytes/bw) in us */
  double tile_intensity;          /* 2*BM*BN / ((BM+BN)*elt): LDS-fill AI */
  int32_t bound;                  /* tx_bound */

  /* loop_split pass: for (k = 0; k < K; k += BK) with the predicate
   * `k > K - BK` (the step that needs a mask) split at k_split:
   *   [0, k_split)  k_main_steps unmasked steps,
   *   [k_split, K)  one peeled masked step of k_tail elements (0 = none). */
  int64_t k_split;
  int32_t k_main_steps;
  int32_t k_tail;
  /* Tile grid, and the extent of the last (masked) tile row / column;
   * 0 when M (N) is a multiple of the tile. */
  int32_t m_tiles, n_tiles;
  int32_t m_edge, n_edge;

  /* mi355x_dot pass: kernel choice and launch shape. */
  int32_t kernel; /* tx_kernel */
  int32_t split_k;
  int32_t grid_x, grid_y, grid_z;
  int32_t block_threads;
  int64_t workspace_bytes; /* device scratch the launch needs (0 = none) */
  int32_t passes_run;      /* number of passes the pipeline ran */
  /* Tile rows per group of the XCD-aware tile order (tiles of one XCD walk
   * group_m tile rows at a time); any value >= 1 gives the same result. */
  int32_t group_m;
};

/* Validate `desc`, run the plan pipeline and fill `plan`. */
TX_API int tx_dot_plan_create(const tx_dot_desc *desc, tx_dot_plan *plan);

/* Enqueue the planned dot on `stream`.  `scale_a`/`scale_b` are required for
 * the scaled modes and ignored otherwise: fp32 arrays for TX_SCALE_ROWCOL and
 * TX_SCALE_BLOCK128, uint8 e8m0 arrays for TX_SCALE_MX32.  `workspace`
 * must hold plan->workspace_bytes bytes when that is non-zero, and be
 * zero-filled before its first use: every workspace starts with a 64 KiB
 * region of the W8A8 decode kernel's arrival counters, which every completed
 * decode launch leaves at zero again and no other kernel writes (the MX
 * upcast of TX_KERNEL_GEMM_MX_BF16 plans goes after it).  So one workspace,
 * zeroed once, serves every plan in turn; the rest of it needs no particular
 * contents.  Launches that may overlap in time (different streams) must not
 * share a workspace. */
TX_API int tx_dot_launch(const tx_dot_plan *plan, const void *A, const void *B,
                         void *C, const void *scale_a, const void *scale_b,
                         void *workspace, size_t workspace_bytes, void *stream);

/* No counterpart in the reference: a variant of tx_dot_launch for callers
 * that cannot allocate device memory (code under HIP graph capture, serving
 * loops and harnesses that forbid hipMalloc).  It takes no workspace: the
 * scratch the planned kernels need (the decode kernels' split-K arrival
 * counters and their int32 or fp32 partials, the MX operand upcast to bf16,
 * the tiles' split-K partials) lives in one
 * static device array of TX_NOALLOC_SCRATCH_BYTES per GPU, held from the
 * library's load on that GPU until the process ends, and the call allocates
 * nothing.  A split-K tile plan whose partials do not fit runs unsplit (the
 * same dot: one K range a tile, fp32 sums in another order).  Any other plan
 * whose workspace does not fit (decode: more than TX_NOALLOC_SCRATCH_BYTES;
 * upcast: more than that less the 64 KiB counter region, which the upcast
 * never touches) returns TX_ERR_WORKSPACE.  Every
 * call on one GPU shares that GPU's array, which keeps the last call's
 * contents: calls that may overlap in time on one GPU (different streams)
 * race on it.  The counters are zero when the library loads and every
 * completed launch leaves them at zero; nothing else needs initial
 * contents. */
#define TX_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
TX_API int tx_dot_launch_noalloc(const tx_dot_plan *plan, const void *A, const void *B,
                                 void *C, const void *scale_a, const void *scale_b,
                                 void *stream);

/* Message for the calling thread's last non-zero status ("" if none). */
TX_API const char *tx_get_last_error(void);
/* Name of a tx_kernel value ("?" if unknown). */
TX_API const char *tx_kernel_name(int32_t kernel);
/* 1 if a gfx950 device is visible to this process, else 0.  Never throws. */
TX_API int tx_device_available(void);

#ifdef __cplusplus
}
#endif

#endif /* TRITON_EXT_AMD_TX_DOT_H */
