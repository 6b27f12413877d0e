// MX operand upcast for gfx950: the first half of tl.dot_scaled with one
// bf16 operand.  Triton states the semantics (T:language/core.py:2072-2076):
// the microscaled operand is upcast to bf16, then an ordinary bf16 dot runs.
// This kernel writes that upcast into a workspace; the 256x256 bf16 tile
// then reads it as its A or B.
//
//   element  x = decode(code) * 2^(s - 127)   (s = 255: NaN)
//   output   bf16 round-to-nearest-even of x, computed as
//            f32_to_bf16_rne(ldexp(decode(code), s - 127))
// decode: e4m3 (OCP: S.1111.111 is NaN, no inf), e5m2 (the top byte of an
// fp16, inf and NaN included), e2m1 (+-{0, .5, 1, 1.5, 2, 3, 4, 6}).  The
// decoded value and its power-of-two scaling are exact in fp32 except past
// fp32's range, so the one rounding is the bf16 one.
//
// Layouts (elements row-major, e2m1 packed two per byte along K, even K in
// the low nibble):
//   B side: src [K][N] (e2m1: [K/2][N] bytes, ld = bytes per packed row),
//           scales [N][K/32]; dst bf16 [K][N], ld N.
//   A side: src [M][K] (e2m1: [M][K/2] bytes), scales [M][K/32]; dst bf16
//           [M][K], ld K.  A thread takes 16 K of one row (one scale).
// The job is streaming (read codes, write 2 bytes per element): HBM-bound,
// with 16-byte loads and 16-byte stores.
#pragma once

#include "tile_common.h"

namespace txk {

struct UpcastArgs {
  const uint8_t *src;
  const uint8_t *scale;
  uint16_t *dst;
  int64_t rows, cols; // of the dst (B side: K x N; A side: M x K)
  int64_t ld_src;     // bytes per src row (e2m1 B: per packed row)
  int64_t ld_scale;   // K / 32
  int32_t fmt;        // 0 e4m3, 1 e5m2, 4 e2m1 (MFMA format codes)
};

__device__ __forceinline__ float mx_decode(uint32_t c, int fmt) {
  if (fmt == 4) { // e2m1: bias 1, subnormal 0.5 m
    const uint32_t e = (c >> 1) & 3, m = c & 1;
    const float v = e == 0 ? 0.5f * (float)m : __builtin_amdgcn_ldexpf(1.f + 0.5f * (float)m, (int)e - 1);
    return (c & 8) ? -v : v;
  }
  if (fmt == 1) // e5m2: the top byte of an fp16
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(c << 8));
  const uint32_t e = (c >> 3) & 15, m = c & 7;
  if (e == 15 && m == 7)
    return __builtin_nanf("");
  const float v = e == 0 ? (float)m * 0x1p-9f : __builtin_amdgcn_ldexpf(1.f + m * 0.125f, (int)e - 7);
  return (c & 0x80) ? -v : v;
}

__device__ __forceinline__ uint16_t mx_upcast1(uint32_t c, int fmt, uint32_t s) {
  const float v = mx_decode(c, fmt);
  const float x = s == 255 ? __builtin_nanf("") : __builtin_amdgcn_ldexpf(v, (int)s - 127);
  return f32_to_bf16_rne(x);
}

// B side: dst[k][n] = upcast(B[k][n] * 2^(scale[n][k/32] - 127)).  A
// thread owns COLS columns and RUN consecutive source rows inside one 32-K
// scale group, so it loads its COLS scale bytes once: fp8 16 columns x 8
// rows, e2m1 8 columns x 4 packed rows (8 K).  Neighbouring threads take
// neighbouring column groups (coalesced 16- / 8-byte loads, 32- / 16-byte
// stores per row).
template <int FMT>
__global__ void __launch_bounds__(256) mx_upcast_b_kernel(UpcastArgs p) {
  constexpr int COLS = FMT == 4 ? 8 : 16; // columns per thread
  constexpr int RUN = FMT == 4 ? 4 : 8;   // source rows per thread
  constexpr int KR = FMT == 4 ? 2 : 1;    // K rows per source row
  const int64_t groups = p.cols / COLS;
  const int64_t srows = p.rows / KR; // source rows
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (srows / RUN) * groups)
    return;
  const int64_t r0 = (t / groups) * RUN, n0 = (t % groups) * COLS;
  const int64_t kg = r0 * KR / 32; // the scale group of all RUN rows
  uint32_t sc[COLS];
#pragma unroll
  for (int i = 0; i < COLS; ++i)
    sc[i] = p.scale[(n0 + i) * p.ld_scale + kg];
  uint8_t code[RUN][16];
#pragma unroll
  for (int r = 0; r < RUN; ++r) {
    const uint8_t *src = p.src + (r0 + r) * p.ld_src + n0;
    if constexpr (FMT == 4)
      *reinterpret_cast<uint64_t *>(code[r]) = *reinterpret_cast<const uint64_t *>(src);
    else
      *reinterpret_cast<u32x4 *>(code[r]) = *reinterpret_cast<const u32x4 *>(src);
  }
#pragma unroll
  for (int r = 0; r < RUN; ++r) {
#pragma unroll
    for (int h = 0; h < KR; ++h) {
      uint16_t out[16];
#pragma unroll
      for (int i = 0; i < COLS; ++i) {
        const uint32_t c = FMT == 4 ? (h ? code[r][i] >> 4 : code[r][i] & 15) : code[r][i];
        out[i] = mx_upcast1(c, FMT, sc[i]);
      }
      uint16_t *d = p.dst + ((r0 + r) * KR + h) * p.cols + n0;
#pragma unroll
      for (int q = 0; q < COLS / 8; ++q)
        reinterpret_cast<u32x4 *>(d)[q] = *reinterpret_cast<const u32x4 *>(&out[8 * q]);
    }
  }
}

// A side: dst[m][k] = upcast(A[m][k] * 2^(scale[m][k/32] - 127)).
template <int FMT>
__global__ void __launch_bounds__(256) mx_upcast_a_kernel(UpcastArgs p) {
  const int64_t groups = p.cols / 16; // 16 K per thread
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= p.rows * groups)
    return;
  const int64_t m = t / groups, k0 = (t % groups) * 16;
  const uint32_t s = p.scale[m * p.ld_scale + k0 / 32];
  uint8_t code[16];
  if constexpr (FMT == 4)
    *reinterpret_cast<uint64_t *>(code) =
        *reinterpret_cast<const uint64_t *>(p.src + m * p.ld_src + k0 / 2);
  else
    *reinterpret_cast<u32x4 *>(code) =
        *reinterpret_cast<const u32x4 *>(p.src + m * p.ld_src + k0);
  uint16_t out[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t c = FMT == 4 ? (i & 1 ? code[i / 2] >> 4 : code[i / 2] & 15) : code[i];
    out[i] = mx_upcast1(c, FMT, s);
  }
  uint16_t *d = p.dst + m * p.cols + k0;
  reinterpret_cast<u32x4 *>(d)[0] = *reinterpret_cast<const u32x4 *>(&out[0]);
  reinterpret_cast<u32x4 *>(d)[1] = *reinterpret_cast<const u32x4 *>(&out[8]);
}

} // namespace txk
