/*
 * Host-side analyses behind the "loop_split" and "arith_intensity"
 * extensions.  Both are plain functions of integers; the extension passes
 * apply them to a tx_dot_plan, and they are exported so that callers (and
 * the tests) can use them directly.
 */
#ifndef TRITON_EXT_AMD_TX_PASSES_H
#define TRITON_EXT_AMD_TX_PASSES_H

#include <stdint.h>

#include "tx_dot.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------
 * loop_split (libloop_split.so)
 *
 * Replaces LoopBisect::bisect, R:pass/LoopSplit/LoopSplit.cpp:125-197, for a
 * loop `for (iv = lo; iv < hi; iv += step)` whose body tests
 * `iv <pred> c` (or `c <pred> iv` when iv_on_rhs) with c loop-invariant.
 * The loop becomes [lo, midp) + [midp, hi') with the predicate folded to
 * `first_value` in the first loop and `second_value` in the second
 * (R:pass/LoopSplit/LoopSplit.cpp:179-193).
 *
 * Semantics follow the mathematics, not the reference's arithmetic, where the
 * two differ: midp is the first iteration value at which the predicate
 * changes, rounded up to the iteration grid and clamped to the iteration
 * range; an operand on the left swaps the comparison (c < iv == iv > c) rather
 * than negating it.  In the reference, sgt/sge at step 1 split one iteration
 * early, the step rounding overshoots by a full step when (midp-lo) % step == 0
 * and bounds are not clamped.
 * ---------------------------------------------------------------------- */

typedef enum tx_cmp_pred {
  /* Values follow arith::CmpIPredicate's order. */
  TX_CMP_EQ = 0,
  TX_CMP_NE = 1,
  TX_CMP_SLT = 2,
  TX_CMP_SLE = 3,
  TX_CMP_SGT = 4,
  TX_CMP_SGE = 5,
  TX_CMP_ULT = 6,
  TX_CMP_ULE = 7,
  TX_CMP_UGT = 8,
  TX_CMP_UGE = 9,
} tx_cmp_pred;

typedef struct tx_loop_split {
  int32_t split;        /* 1 if the loop is split (both halves may be empty) */
  int32_t first_value;  /* predicate value folded into [lo, midp)           */
  int32_t second_value; /* predicate value folded into [midp, hi)           */
  int32_t reserved;
  int64_t midp;         /* first iteration value of the second loop         */
  int64_t first_trips;  /* iterations in [lo, midp)                         */
  int64_t second_trips; /* iterations in [midp, hi)                         */
} tx_loop_split;

/* Returns TX_OK and fills `out`; out->split = 0 (with TX_OK) when the loop is
 * not splittable: step <= 0 (the reference rejects it too,
 * R:pass/LoopSplit/LoopSplit.cpp:130-138), an eq/ne predicate (not in
 * CmpTypeMap, :35-44), or an unsigned predicate whose operands are not all
 * non-negative (then the signed and unsigned orders differ and the predicate
 * need not be monotone over the loop).  `bits` is the IV width (1..64);
 * lo, hi and c must fit in it as signed values.  TX_ERR_INVALID for a NULL
 * out or bad width. */
TX_API int tx_loop_split_plan(int64_t lo, int64_t hi, int64_t step,
                              int32_t pred, int64_t c, int32_t iv_on_rhs,
                              int32_t bits, tx_loop_split *out);

/* The K loop of a tiled dot: for (k = 0; k < K; k += bk) with the mask
 * predicate `k > K - bk`.  Fills the plan fields k_split, k_main_steps and
 * k_tail by calling tx_loop_split_plan. */
TX_API int tx_loop_split_k(int64_t K, int32_t bk, int64_t *k_split,
                           int32_t *k_main_steps, int32_t *k_tail);

/* ------------------------------------------------------------------------
 * arith_intensity (libarith_intensity.so)
 *
 * Absent from the reference snapshot (named only in the task statement).
 * FLOPs = 2*M*N*K; bytes = A + B + C + scales, each read or written once;
 * ridge = peak_flops / peak_bw; bound = MFMA if intensity > ridge.
 * MI355X peaks (dense, public): bf16/fp16 2.5166 PFLOP/s, int8 and fp8
 * 5.0332 P(FL)OP/s, fp4 10.0664 PFLOP/s, HBM3E 8.0 TB/s.
 * ---------------------------------------------------------------------- */

typedef struct tx_ai_report {
  double flops, bytes, intensity;
  double peak_flops, peak_bw, ridge;
  double roofline_us;
  double tile_intensity;
  int32_t bound;
  int32_t block_m, block_n, block_k; /* recommended tile */
} tx_ai_report;

/* Element size in bytes of a tx_dtype (0 for an unknown value and for the
 * sub-byte TX_F4E2M1). */
TX_API int32_t tx_dtype_size(int32_t dtype);
/* Element size in bits of a tx_dtype (0 for an unknown value). */
TX_API int32_t tx_dtype_bits(int32_t dtype);
/* MI355X dense peak FLOP/s (or OP/s) for a product of `dtype` operands. */
TX_API double tx_mi355x_peak_flops(int32_t dtype);
/* MI355X HBM3E peak bytes/s. */
TX_API double tx_mi355x_peak_bw(void);
/* Classify a dot and recommend a tile (desc->block_* if non-zero).  The
 * 256-wide tiles address A and B through 32-bit buffer offsets, so an
 * operand spanning 2 GiB or more (tx_dot_operand_spans) gets a 128x128 tile,
 * whose loads use 64-bit addresses. */
TX_API int tx_arith_intensity(const tx_dot_desc *desc, tx_ai_report *out);
/* Bytes from A's first element to one past its last, and the same for B,
 * with desc's strides (0 = packed; B [N][K] under TX_FLAG_B_KMAJOR; e2m1
 * packed two per byte along K).  Saturates at INT64_MAX.  TX_ERR_INVALID for
 * a NULL argument or an unknown dtype. */
TX_API int tx_dot_operand_spans(const tx_dot_desc *desc, int64_t *a_bytes, int64_t *b_bytes);
/* Largest operand span (bytes, exclusive) the 32-bit-offset tiles take. */
#define TX_SPAN32_LIMIT ((int64_t)1 << 31)
/* Split-K factor of a dot on the 256x256 tiles: with fewer than half as many
 * tiles as the 256 CUs, K is cut into S ranges of whole K steps, the
 * workgroups (tile, range) store fp32 / int32 partial sums, and a second
 * kernel adds them in range order and applies the epilogue.  S is the
 * largest power of two up to 16 with tiles * S <= 256 and at least 8 K steps
 * a range; 1 (no split) otherwise. */
TX_API int32_t tx_gemm_split_k(int64_t tiles, int64_t ksteps);
/* Row stride (elements) of a B operand that tl.dot_scaled with one bf16 side
 * upcasts to bf16 in the workspace: N rounded up to 16 columns, so every row
 * starts 16-byte aligned for the bf16 tile.  (An upcast A is packed: K.) */
#define TX_MX_UPCAST_LD(n) ((((int64_t)(n)) + 15) / 16 * 16)

#ifdef __cplusplus
}
#endif

#endif /* TRITON_EXT_AMD_TX_PASSES_H */
