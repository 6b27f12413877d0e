// loop_split extension: libloop_split.so.
//
// The reference's LoopSplit pass (R:pass/LoopSplit/LoopSplit.cpp) rewrites an
// scf.for whose body compares the induction variable with a loop-invariant
// value into two consecutive loops with the comparison folded to a constant
// in each (:125-197).  For the tiled dot that is the K loop: the comparison
// `k > K - BK` marks the one step whose loads need a mask, and splitting the
// loop gives an unmasked main loop over full K tiles plus a peeled masked
// tail.  Here the split point is computed on the host and drives the
// kernel's loop bounds (tx_dot_plan.k_split / k_main_steps / k_tail).
//
// Split-point arithmetic (the reference's is in :156-174): the predicate
// `iv < t`-style threshold t is c for slt/sge and c + 1 for sle/sgt; the
// second loop starts at the first iteration value >= t, i.e.
// lo + ceil((t - lo) / step) * step, clamped to the iteration range.

#include "triton_ext/TritonExtPassInfra.h"
#include "triton_ext/tx_dot.h"
#include "triton_ext/tx_passes.h"

#include <cstdint>

namespace {

typedef __int128 i128;

i128 ceilDiv(i128 a, i128 b) { // b > 0
  if (a >= 0)
    return (a + b - 1) / b;
  return -((-a) / b);
}

bool fitsSigned(int64_t v, int bits) {
  if (bits >= 64)
    return true;
  int64_t lim = (int64_t)1 << (bits - 1);
  return v >= -lim && v < lim;
}

// Predicate with the IV moved to the left-hand side: `c P iv` == `iv P' c`
// with P' the operand-swapped predicate.
int32_t swapOperands(int32_t p) {
  switch (p) {
  case TX_CMP_SLT: return TX_CMP_SGT;
  case TX_CMP_SLE: return TX_CMP_SGE;
  case TX_CMP_SGT: return TX_CMP_SLT;
  case TX_CMP_SGE: return TX_CMP_SLE;
  case TX_CMP_ULT: return TX_CMP_UGT;
  case TX_CMP_ULE: return TX_CMP_UGE;
  case TX_CMP_UGT: return TX_CMP_ULT;
  case TX_CMP_UGE: return TX_CMP_ULE;
  default: return p;
  }
}

} // namespace

extern "C" int tx_loop_split_plan(int64_t lo, int64_t hi, int64_t step,
                                  int32_t pred, int64_t c, int32_t iv_on_rhs,
                                  int32_t bits, tx_loop_split *out) {
  if (!out || bits < 1 || bits > 64)
    return TX_ERR_INVALID;
  *out = tx_loop_split{};
  if (!fitsSigned(lo, bits) || !fitsSigned(hi, bits) || !fitsSigned(c, bits))
    return TX_ERR_INVALID;
  if (step <= 0)
    return TX_OK; // not splittable (R:pass/LoopSplit/LoopSplit.cpp:130-138)
  int32_t p = iv_on_rhs ? swapOperands(pred) : pred;
  bool isUnsigned = p >= TX_CMP_ULT && p <= TX_CMP_UGE;
  if (isUnsigned) {
    // Over non-negative values the unsigned order equals the signed one;
    // otherwise the predicate need not be monotone in iv: decline.
    if (lo < 0 || hi < 0 || c < 0)
      return TX_OK;
    p = p - TX_CMP_ULT + TX_CMP_SLT;
  }
  i128 t;
  int32_t firstValue;
  switch (p) {
  case TX_CMP_SLT: t = c; firstValue = 1; break;
  case TX_CMP_SGE: t = c; firstValue = 0; break;
  case TX_CMP_SLE: t = (i128)c + 1; firstValue = 1; break;
  case TX_CMP_SGT: t = (i128)c + 1; firstValue = 0; break;
  default: return TX_OK; // eq / ne: not in the reference's CmpTypeMap
  }
  i128 trips = hi > lo ? ceilDiv((i128)hi - lo, step) : 0;
  i128 first = ceilDiv(t - lo, step);
  if (first < 0)
    first = 0;
  if (first > trips)
    first = trips;
  int64_t midp;
  if (trips == 0 || first == 0)
    midp = lo;
  else if (first == trips)
    midp = hi; // the whole loop stays in the first half
  else
    midp = (int64_t)((i128)lo + first * step);
  out->split = 1;
  out->first_value = firstValue;
  out->second_value = !firstValue;
  out->midp = midp;
  out->first_trips = (int64_t)first;
  out->second_trips = (int64_t)(trips - first);
  return TX_OK;
}

extern "C" int tx_loop_split_k(int64_t K, int32_t bk, int64_t *k_split,
                               int32_t *k_main_steps, int32_t *k_tail) {
  if (!k_split || !k_main_steps || !k_tail || K < 0 || bk <= 0)
    return TX_ERR_INVALID;
  // for (k = 0; k < K; k += bk) { if (k > K - bk) <masked load> }
  tx_loop_split s;
  int rc = tx_loop_split_plan(0, K, bk, TX_CMP_SGT, K - bk, 0, 64, &s);
  if (rc != TX_OK)
    return rc;
  *k_split = s.midp;
  *k_main_steps = (int32_t)s.first_trips;
  *k_tail = (int32_t)(K - s.midp);
  return TX_OK;
}

namespace {

// Pass body: plan the K loop and the M/N edge tiles of one dot.
int txLoopSplitRun(tx_dot_plan *plan) {
  tx_dot_desc &d = plan->desc;
  if (d.block_m <= 0 || d.block_n <= 0 || d.block_k <= 0)
    return TX_ERR_INVALID; // tiles are chosen by arith_intensity first
  if (d.flags & TX_FLAG_NO_LOOP_SPLIT) {
    plan->k_split = 0;
    plan->k_main_steps = 0;
    plan->k_tail = (int32_t)d.K;
  } else {
    int rc = tx_loop_split_k(d.K, d.block_k, &plan->k_split,
                             &plan->k_main_steps, &plan->k_tail);
    if (rc != TX_OK)
      return rc;
  }
  plan->m_tiles = (int32_t)((d.M + d.block_m - 1) / d.block_m);
  plan->n_tiles = (int32_t)((d.N + d.block_n - 1) / d.block_n);
  plan->m_edge = (int32_t)(d.M % d.block_m);
  plan->n_edge = (int32_t)(d.N % d.block_n);
  plan->passes_run += 1;
  return TX_OK;
}

} // namespace

#define TRITON_EXT_ARG "triton-loop-split"
#define TRITON_EXT_RUN txLoopSplitRun
#include "../../infra/TritonExtPass.inc"
