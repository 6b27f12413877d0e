/*
 * Fused attention forward on MI355X (gfx950): plan + launch C-ABI.
 *
 * The computation is the forward of the reference's fused-attention
 * tutorial, the kernel whose K/V loop the LoopSplit pass exists to split
 * (R:pass/LoopSplit/06-fused-attention.py:44-93 `_attn_fwd_inner`,
 * :181-239 `_attn_fwd`, :583-640 `_attention.forward`):
 *
 *     per (z, h) and block of BLOCK_M query rows m:
 *       m_i = -inf, l_i = 1, acc = 0, qk_scale = sm_scale * 1.44269504
 *       for start_n in range(0, N_CTX, BLOCK_N):       # split by LoopSplit at
 *         qk = q @ k[start_n:+BLOCK_N].T                # causal_start
 *         if start_n >= causal_start:                   # on-band: masked
 *           qk = qk * qk_scale + where(m >= start_n + n, 0, -1e6)
 *           m_ij = max(m_i, rowmax(qk));  qk -= m_ij
 *         else:                                         # off-band
 *           m_ij = max(m_i, rowmax(qk) * qk_scale);  qk = qk * qk_scale - m_ij
 *         p = exp2(qk);  alpha = exp2(m_i - m_ij)
 *         l_i = l_i * alpha + rowsum(p);  acc = acc * alpha + p.to(fp16) @ v
 *         m_i = m_ij
 *       M[m] = m_i + log2(l_i);  O[m] = (acc / l_i).to(fp16)
 *
 * causal_start is start_m * BLOCK_M for causal attention and N_CTX
 * otherwise; the loop is run as LoopSplit leaves it: an unmasked main loop
 * over [0, causal_start) and the masked on-band blocks.  Blocks that lie
 * entirely past the diagonal add exactly zero (p = 0, alpha = 1 while
 * |qk * qk_scale| < 1e6 - |m_i|) and are not run.
 *
 * q, k, v, o are [Z][H][N_CTX][HEAD_DIM] fp16 or bf16 with HEAD_DIM contiguous and
 * the given element strides; M is fp32 [Z * H][N_CTX] (the tutorial's
 * logsumexp in base 2, saved for the backward).  All device pointers; errors
 * by return code and tx_get_last_error() (tx_dot.h).
 *
 * dtype TX_F8E5M2 is the tutorial's fp8 provider (:774-779, :81-82): q, k, o
 * e5m2 [Z][H][N_CTX][HEAD_DIM] as above; v e5m2 stored key-contiguous, as
 * v.permute(0, 1, 3, 2).contiguous().permute(0, 1, 3, 2) leaves it, i.e.
 * [Z][H][HEAD_DIM][N_CTX] with v_sm the stride between head-dim rows
 * (default N_CTX); p and o are rounded to e5m2 to nearest even.
 */
#ifndef TRITON_EXT_AMD_TX_ATTN_H
#define TRITON_EXT_AMD_TX_ATTN_H

#include "triton_ext/tx_dot.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct tx_attn_desc {
  int64_t Z, H, N_CTX;
  int32_t head_dim; /* 16, 32, 64, 128 or 256 */
  int32_t dtype;    /* TX_F16 (the tutorial's), TX_BF16 or TX_F8E5M2 for q, k, v, o */
  int32_t causal;   /* 0 or 1 */
  float sm_scale;
  /* element strides (batch, head, row) of q, k, v, o; 0 = packed; each a
   * multiple of 16 bytes (e5m2 v: (batch, head, head-dim row)) */
  int64_t q_sz, q_sh, q_sm;
  int64_t k_sz, k_sh, k_sm;
  int64_t v_sz, v_sh, v_sm;
  int64_t o_sz, o_sh, o_sm;
  /* BLOCK_M x BLOCK_N, one of the tutorial's autotuned configs
   * (R:pass/LoopSplit/06-fused-attention.py:145-159): BLOCK_M 64 or 128 by
   * BLOCK_N 32 or 64 (not 128 x 32 at head dims below 64, or below 128
   * for fp8 e5m2); 0 = default (128, 64).  The
   * blocks fix the on-band split (causal_start = start_m * BLOCK_M) and the
   * online softmax's key blocks, so they select the rounding of the result
   * exactly as the tutorial's config does. */
  int32_t block_m, block_n;
} tx_attn_desc;

typedef struct tx_attn_plan {
  tx_attn_desc desc; /* resolved copy (strides and blocks filled in) */
  double flops;      /* 4 * Z * H * N_CTX^2 * HEAD_DIM (x 1/2 causal) */
  double bytes;      /* q, k, v read once, o and M written once */
  float qk_scale;    /* sm_scale * 1.44269504, in fp32 as the kernel has it */
  int32_t m_blocks;  /* N_CTX / block_m programs per (z, h) */
  int32_t grid_x, block_threads;
  int32_t reserved;
} tx_attn_plan;

/* Validate `desc` and fill `plan`.  TX_ERR_UNSUPPORTED unless dtype is
 * TX_F16, TX_BF16 or TX_F8E5M2 with head_dim 16, 32, 64, 128 or 256, the
 * blocks one of the implemented configs (BLOCK_M 64 or 128 by BLOCK_N 32 or
 * 64, at every head_dim) and N_CTX a multiple of BLOCK_M (the tutorial's block pointers assume whole
 * blocks).  p is rounded to q's type to nearest even before p @ v, as
 * compiled Triton does. */
TX_API int tx_attn_fwd_plan(const tx_attn_desc *desc, tx_attn_plan *plan);

/* Enqueue the forward on `stream` (a hipStream_t, NULL = null stream). */
TX_API int tx_attn_fwd_launch(const tx_attn_plan *plan, const void *q, const void *k,
                              const void *v, void *o, float *M, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* TRITON_EXT_AMD_TX_ATTN_H */
