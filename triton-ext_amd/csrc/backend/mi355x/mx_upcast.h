// MX operand upcast for gfx950: the first half of tl.dot_scaled with one
// bf16 operand.  Triton states the semantics (T:language/core.py:2072-2076):
// the microscaled operand is upcast to bf16, then an ordinary bf16 dot runs.
// This kernel writes that upcast into a workspace; the 256x256 bf16 tile
// then reads it as its A or B.
//
//   element  x = decode(code) * 2^(s - 127)   (s = 255: NaN)
//   output   bf16 round-to-nearest-even of x: for scale exponents 17..239
//            by v_cvt_scalef32_pk_bf16_* (exact there, see mx_cvt_pair),
//            else as f32_to_bf16_rne(ldexp(decode(code), s - 127))
// decode: e4m3 (OCP: S.1111.111 is NaN, no inf), e5m2 (the top byte of an
// fp16, inf and NaN included), e2m1 (+-{0, .5, 1, 1.5, 2, 3, 4, 6}).  The
// decoded value and its power-of-two scaling are exact in fp32 except past
// fp32's range, so the one rounding is the bf16 one.
//
// Layouts (elements row-major, e2m1 packed two per byte along K, even K in
// the low nibble):
//   B side: src [K][N] (e2m1: [K/2][N] bytes, ld = bytes per packed row),
//           scales [N][K/32]; dst bf16 [K][N], ld N rounded up to 16.  A
//           thread takes 16 columns; in the group that crosses N it reads
//           only the bytes and scales of columns < N and writes zeros past
//           N (the bf16 tile drops those columns).
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
  int64_t ld_dst;     // dst elements per row (B side: N rounded up to 16; A side: K)
  int64_t ld_src;     // bytes per src row (e2m1 B: per packed row)
  int64_t ld_scale;   // K / 32 (K / 16 for e4m3 scales)
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


// Hardware pair conversion: v_cvt_scalef32_pk_bf16_{fp8,bf8,fp4} decodes
// two elements (bytes 2w, 2w + 1 of `src`, or byte `sel`'s two e2m1 nibbles)
// and multiplies by one fp32 scale.  Used only where the scale exponent lies
// in [17, 239]: there every result is a normal bf16 with at most 4
// significant bits -- exact, so the instruction's rounding never applies --
// and a zero code stays zero.  Other scales (subnormal results, overflow,
// 0xFF) take mx_upcast1.  Returns the two bf16 as (lo, hi) halves.
constexpr uint32_t kHwScaleLo = 17, kHwScaleHi = 239;
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
template <int FMT, int SEL>
__device__ __forceinline__ uint32_t mx_cvt_pair(uint32_t src, float scale) {
  bf16x2_t r;
  if constexpr (FMT == 0)
    r = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(src, scale, SEL != 0);
  else if constexpr (FMT == 1)
    r = __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(src, scale, SEL != 0);
  else
    r = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(src, scale, SEL);
  return __builtin_bit_cast(uint32_t, r);
}

// Scales: e8m0 per 32 K (MX), or e4m3 per 16 K (NV: the fp8e4nv scale
// tensors of tl.dot_scaled).  An e4m3 scale is a plain multiplier; e2m1
// times e4m3 has at most 6 significant bits, so the bf16 product is exact.
// The pair conversion takes only the exponent of its fp32 scale (it serves
// e8m0's powers of two), so e4m3 scales, which carry mantissa bits, always
// take the element path.
template <bool NV> struct ScaleKind {
  static constexpr int GROUP = NV ? 16 : 32;
  // the pair conversion applies (exact products, see mx_cvt_pair)
  __device__ __forceinline__ static bool hw(uint32_t s) {
    return !NV && s >= kHwScaleLo && s <= kHwScaleHi;
  }
  __device__ __forceinline__ static float factor(uint32_t s) {
    return NV ? mx_decode(s, 0) : __builtin_amdgcn_ldexpf(1.0f, (int)s - 127);
  }
  __device__ __forceinline__ static uint16_t one(uint32_t c, int fmt, uint32_t s) {
    return NV ? f32_to_bf16_rne(mx_decode(c, fmt) * mx_decode(s, 0)) : mx_upcast1(c, fmt, s);
  }
};

// B side: dst[k][n] = upcast(B[k][n] * 2^(scale[n][k/32] - 127)).  A
// thread owns 16 columns and the source rows of 8 consecutive K inside one
// 32-K scale group (fp8 8 rows, e2m1 4 packed rows), so it loads its 16
// scale bytes once.  Neighbouring threads take neighbouring column groups
// (coalesced 16-byte loads and 32-byte row stores).  B's scales vary along a row, so the pair conversion
// runs on K pairs of one column: fp8 bytes of rows k, k + 1 are paired by
// v_perm_b32, e2m1 bytes hold K pairs already; results are re-paired into
// row order by v_perm_b32.
template <int FMT, bool NV = false>
__global__ void __launch_bounds__(256) mx_upcast_b_kernel(UpcastArgs p) {
  typedef ScaleKind<NV> SK;
  constexpr int COLS = 16;              // columns per thread
  constexpr int RUN = FMT == 4 ? 4 : 8; // source rows per thread (8 K)
  constexpr int KR = FMT == 4 ? 2 : 1;  // K rows per source row
  const int64_t groups = (p.cols + COLS - 1) / COLS;
  const int64_t srows = p.rows / KR; // source rows
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (srows / RUN) * groups)
    return;
  const int64_t r0 = (t / groups) * RUN, n0 = (t % groups) * COLS;
  const int64_t kg = r0 * KR / SK::GROUP; // the scale group of all RUN rows
  // valid columns of this group: COLS except in the group that crosses N
  const int ncol = p.cols - n0 < COLS ? (int)(p.cols - n0) : COLS;
  uint32_t sc[COLS];
  bool hw = true;
#pragma unroll
  for (int i = 0; i < COLS; ++i) {
    sc[i] = p.scale[(n0 + (i < ncol ? i : 0)) * p.ld_scale + kg];
    hw = hw && SK::hw(sc[i]);
  }
  uint32_t w[RUN][COLS / 4]; // source dwords: row r, columns 4 q .. +3
  if (ncol == COLS) {
#pragma unroll
    for (int r = 0; r < RUN; ++r) {
      const u32x4 v = *reinterpret_cast<const u32x4 *>(p.src + (r0 + r) * p.ld_src + n0);
#pragma unroll
      for (int q = 0; q < 4; ++q)
        w[r][q] = v[q];
    }
  } else { // the bytes of columns < N only (the row may end at N)
#pragma unroll
    for (int r = 0; r < RUN; ++r)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t x = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b)
          if (4 * q + b < ncol)
            x |= (uint32_t)p.src[(r0 + r) * p.ld_src + n0 + 4 * q + b] << (8 * b);
        w[r][q] = x;
      }
  }
  // bf16 pair words of columns >= N (in the crossing group) become zero
  uint32_t keep[COLS / 2];
#pragma unroll
  for (int c = 0; c < COLS; c += 2)
    keep[c / 2] = (c < ncol ? 0xFFFFu : 0u) | (c + 1 < ncol ? 0xFFFF0000u : 0u);
  auto store_row = [&](int64_t k, const uint32_t (&o)[COLS / 2]) {
    uint16_t *d = p.dst + k * p.ld_dst + n0;
#pragma unroll
    for (int q = 0; q < COLS / 8; ++q)
      reinterpret_cast<u32x4 *>(d)[q] =
          u32x4{o[4 * q] & keep[4 * q], o[4 * q + 1] & keep[4 * q + 1],
                o[4 * q + 2] & keep[4 * q + 2], o[4 * q + 3] & keep[4 * q + 3]};
  };
  if (hw) {
    float sf[COLS];
#pragma unroll
    for (int i = 0; i < COLS; ++i)
      sf[i] = SK::factor(sc[i]);
    if constexpr (FMT == 4) {
      // byte i of a packed row: column n0 + i, K rows 2 r and 2 r + 1
#pragma unroll
      for (int r = 0; r < RUN; ++r) {
        uint32_t lo[COLS / 2], hi[COLS / 2]; // rows 2 r and 2 r + 1, column pairs
#pragma unroll
        for (int c = 0; c < COLS; c += 2) {
          const uint32_t src0 = w[r][c / 4], sel0 = c % 4;
          const uint32_t a = sel0 == 0 ? mx_cvt_pair<4, 0>(src0, sf[c])
                           : mx_cvt_pair<4, 2>(src0, sf[c]);
          const uint32_t b = sel0 == 0 ? mx_cvt_pair<4, 1>(src0, sf[c + 1])
                           : mx_cvt_pair<4, 3>(src0, sf[c + 1]);
          // a = (k, c) | (k + 1, c) << 16, b likewise for column c + 1
          lo[c / 2] = __builtin_amdgcn_perm(b, a, 0x05040100u); // (k, c) | (k, c + 1) << 16
          hi[c / 2] = __builtin_amdgcn_perm(b, a, 0x07060302u); // (k + 1, c) | (k + 1, c + 1) << 16
        }
        store_row(2 * (r0 + r), lo);
        store_row(2 * (r0 + r) + 1, hi);
      }
    } else {
#pragma unroll
      for (int r = 0; r < RUN; r += 2) {
        uint32_t lo[COLS / 2], hi[COLS / 2];
#pragma unroll
        for (int c = 0; c < COLS; c += 2) {
          // bytes (k, c), (k + 1, c), (k, c + 1), (k + 1, c + 1)
          const uint32_t x = w[r][c / 4], y = w[r + 1][c / 4];
          const uint32_t sh = c % 4; // byte of column c within its dword
          const uint32_t pr = __builtin_amdgcn_perm(y, x, (sh) | ((sh + 4) << 8) |
                                                              ((sh + 1) << 16) | ((sh + 5) << 24));
          const uint32_t a = mx_cvt_pair<FMT, 0>(pr, sf[c]);     // (k, c), (k + 1, c)
          const uint32_t b = mx_cvt_pair<FMT, 1>(pr, sf[c + 1]); // (k, c + 1), (k + 1, c + 1)
          lo[c / 2] = __builtin_amdgcn_perm(b, a, 0x05040100u);
          hi[c / 2] = __builtin_amdgcn_perm(b, a, 0x07060302u);
        }
        store_row(r0 + r, lo);
        store_row(r0 + r + 1, hi);
      }
    }
    return;
  }
  // scales outside [17, 239]: element by element
#pragma unroll
  for (int r = 0; r < RUN; ++r) {
#pragma unroll
    for (int h = 0; h < KR; ++h) {
      uint32_t o[COLS / 2];
#pragma unroll
      for (int c = 0; c < COLS; c += 2) {
        uint32_t e[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const uint32_t byte = (w[r][(c + u) / 4] >> (8 * ((c + u) % 4))) & 0xFFu;
          const uint32_t code = FMT == 4 ? (h ? byte >> 4 : byte & 15) : byte;
          e[u] = SK::one(code, FMT, sc[c + u]);
        }
        o[c / 2] = e[0] | (e[1] << 16);
      }
      store_row((r0 + r) * KR + h, o);
    }
  }
}

// A side: dst[m][k] = upcast(A[m][k] * 2^(scale[m][k/32] - 127)).
template <int FMT, bool NV = false>
__global__ void __launch_bounds__(256) mx_upcast_a_kernel(UpcastArgs p) {
  typedef ScaleKind<NV> SK;
  const int64_t groups = p.cols / 16; // 16 K per thread
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= p.rows * groups)
    return;
  const int64_t m = t / groups, k0 = (t % groups) * 16;
  const uint32_t s = p.scale[m * p.ld_scale + k0 / SK::GROUP];
  uint8_t code[16];
  if constexpr (FMT == 4)
    *reinterpret_cast<uint64_t *>(code) =
        *reinterpret_cast<const uint64_t *>(p.src + m * p.ld_src + k0 / 2);
  else
    *reinterpret_cast<u32x4 *>(code) =
        *reinterpret_cast<const u32x4 *>(p.src + m * p.ld_src + k0);
  uint16_t *d = p.dst + m * p.ld_dst + k0;
  if (SK::hw(s)) {
    // neighbouring K share the scale: pairs convert in place (see mx_cvt_pair)
    const float sf = SK::factor(s);
    uint32_t o[8];
    const uint32_t *cw = reinterpret_cast<const uint32_t *>(code);
#pragma unroll
    for (int q = 0; q < (FMT == 4 ? 2 : 4); ++q) {
      if constexpr (FMT == 4) {
        o[4 * q] = mx_cvt_pair<4, 0>(cw[q], sf);
        o[4 * q + 1] = mx_cvt_pair<4, 1>(cw[q], sf);
        o[4 * q + 2] = mx_cvt_pair<4, 2>(cw[q], sf);
        o[4 * q + 3] = mx_cvt_pair<4, 3>(cw[q], sf);
      } else {
        o[2 * q] = mx_cvt_pair<FMT, 0>(cw[q], sf);
        o[2 * q + 1] = mx_cvt_pair<FMT, 1>(cw[q], sf);
      }
    }
    reinterpret_cast<u32x4 *>(d)[0] = u32x4{o[0], o[1], o[2], o[3]};
    reinterpret_cast<u32x4 *>(d)[1] = u32x4{o[4], o[5], o[6], o[7]};
    return;
  }
  uint16_t out[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t c = FMT == 4 ? (i & 1 ? code[i / 2] >> 4 : code[i / 2] & 15) : code[i];
    out[i] = SK::one(c, FMT, s);
  }
  reinterpret_cast<u32x4 *>(d)[0] = *reinterpret_cast<const u32x4 *>(&out[0]);
  reinterpret_cast<u32x4 *>(d)[1] = *reinterpret_cast<const u32x4 *>(&out[8]);
}

} // namespace txk
