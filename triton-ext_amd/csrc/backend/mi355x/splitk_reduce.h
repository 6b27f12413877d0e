// Second kernel of a split-K dot on the 256x256 tiles: C = epilogue(sum of
// the split_k partial sums), the partials added in range order 0, 1, .. so
// the result does not depend on which workgroup finished first.
//
// The tile kernels store range z's 32-bit sums (fp32, or int32 for int8
// operands) at part + z M ldp, row-major with ldp (N rounded up to 4)
// elements a row.  A thread owns one column quad of one row: one 16-byte
// load per range, then one store of the quad (single elements where it
// crosses N).  Epilogues:
//   SPLIT_F32   fp32 C = sum (C += sum under acc);
//   SPLIT_BF16, SPLIT_F16   16-bit C = sum rounded to nearest even;
//   SPLIT_I32   int32 C = sum (C += sum under acc);
//   SPLIT_ROWCOL   W8A8: bf16((float(sum) * sa[m]) * sb[n]), the tile's and
//                  the decode kernels' order, rounded to nearest even.
#pragma once

#include "gemm_tile.h"

namespace txk {

typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;

enum SplitEpilogue { SPLIT_F32 = 0, SPLIT_BF16 = 1, SPLIT_F16 = 2, SPLIT_I32 = 3, SPLIT_ROWCOL = 4 };

struct SplitReduceArgs {
  const uint8_t *part; // [split_k][M][ldp] fp32 / int32
  void *C;
  const float *sa, *sb; // SPLIT_ROWCOL: [M], [N]
  int64_t ldc, ldp;     // row strides in elements
  int32_t M, N, split_k;
  int32_t kind; // SplitEpilogue
  int32_t acc;  // SPLIT_F32 / SPLIT_I32: add to C's contents
};

__global__ void __launch_bounds__(256) splitk_reduce_kernel(SplitReduceArgs p) {
  const int qn = (p.N + 3) / 4;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)p.M * qn)
    return;
  const int m = (int)(idx / qn), n = 4 * (int)(idx % qn);
  const int64_t off = (int64_t)m * p.ldp + n, stride = (int64_t)p.M * p.ldp;
  const bool whole = n + 4 <= p.N;
  if (p.kind == SPLIT_I32 || p.kind == SPLIT_ROWCOL) {
    const i32x4_t *src = reinterpret_cast<const i32x4_t *>(p.part) + off / 4;
    i32x4_t s = src[0];
    for (int z = 1; z < p.split_k; ++z)
      s += src[z * (stride / 4)];
    if (p.kind == SPLIT_I32) {
      int32_t *c = static_cast<int32_t *>(p.C) + (int64_t)m * p.ldc + n;
      if (whole) {
        if (p.acc)
          s += *reinterpret_cast<const i32x4_t *>(c);
        *reinterpret_cast<i32x4_t *>(c) = s;
      } else {
        for (int r = 0; r < 4; ++r)
          if (n + r < p.N)
            c[r] = p.acc ? c[r] + s[r] : s[r];
      }
      return;
    }
    const float sam = p.sa[m];
    float f[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
#pragma clang fp contract(off)
      f[r] = ((float)s[r] * sam) * p.sb[n + r < p.N ? n + r : 0];
    }
    uint16_t *c = static_cast<uint16_t *>(p.C) + (int64_t)m * p.ldc + n;
    if (whole) {
      uint2 w;
      w.x = pk_bf16_rne(f[0], f[1]);
      w.y = pk_bf16_rne(f[2], f[3]);
      *reinterpret_cast<uint2 *>(c) = w;
    } else {
      for (int r = 0; r < 4; ++r)
        if (n + r < p.N)
          c[r] = f32_to_bf16_rne(f[r]);
    }
    return;
  }
  const f32x4_t *src = reinterpret_cast<const f32x4_t *>(p.part) + off / 4;
  f32x4_t s = src[0];
  for (int z = 1; z < p.split_k; ++z)
    s += src[z * (stride / 4)];
  if (p.kind == SPLIT_F32) {
    float *c = static_cast<float *>(p.C) + (int64_t)m * p.ldc + n;
    if (whole) {
      if (p.acc)
        s += *reinterpret_cast<const f32x4_t *>(c);
      *reinterpret_cast<f32x4_t *>(c) = s;
    } else {
      for (int r = 0; r < 4; ++r)
        if (n + r < p.N)
          c[r] = p.acc ? c[r] + s[r] : s[r];
    }
    return;
  }
  const bool bf = p.kind == SPLIT_BF16;
  uint16_t *c = static_cast<uint16_t *>(p.C) + (int64_t)m * p.ldc + n;
  if (whole) {
    uint2 w;
    w.x = bf ? pk_bf16_rne(s[0], s[1]) : pk_f16_rne(s[0], s[1]);
    w.y = bf ? pk_bf16_rne(s[2], s[3]) : pk_f16_rne(s[2], s[3]);
    *reinterpret_cast<uint2 *>(c) = w;
  } else {
    for (int r = 0; r < 4; ++r)
      if (n + r < p.N)
        c[r] = bf ? f32_to_bf16_rne(s[r]) : f32_to_f16_rne(s[r]);
  }
}

} // namespace txk
