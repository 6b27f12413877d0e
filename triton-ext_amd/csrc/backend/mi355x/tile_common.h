// Shared device helpers for the gfx950 tiled-dot kernels: vector types,
// byte-permute transposes, bf16 rounding and the LDS swizzle.
//
// The transposes are __host__ __device__ so the same code is checked on the
// CPU (tests/transpose_host.cpp is a host harness over them).
#pragma once

#include <stdint.h>
#include <string.h>

#ifdef __HIPCC__
#include <hip/hip_runtime.h>
#define TX_HD __host__ __device__ __forceinline__
#else
#define TX_HD static inline
#endif

namespace txk {

// 16 bytes as four dwords; a GCC/Clang vector so a load or store of one is a
// single 128-bit access.
typedef uint32_t u32x4 __attribute__((vector_size(16)));

TX_HD uint32_t get(const u32x4 &v, int i) { return v[i]; }
TX_HD void set(u32x4 &v, int i, uint32_t s) { v[i] = s; }

// v_perm_b32 semantics: the 8 source bytes are {lo bytes 0-3, hi bytes 4-7};
// selector byte i (0..7) picks result byte i.
TX_HD uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_amdgcn_perm(hi, lo, sel);
#else
  uint64_t src = ((uint64_t)hi << 32) | lo;
  uint32_t r = 0;
  for (int i = 0; i < 4; ++i) {
    uint32_t s = (sel >> (8 * i)) & 0xff;
    r |= (uint32_t)((src >> (8 * (s & 7))) & 0xff) << (8 * i);
  }
  return r;
#endif
}

// 8x8 transpose of 16-bit elements.  in[j] holds row j (8 elements, element
// c in 16-bit lane c); out[c] receives column c (element j = in[j][c]).
TX_HD void transpose8x8_b16(const u32x4 *in, u32x4 *out) {
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    u32x4 o;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      uint32_t x = get(in[2 * d], c >> 1), y = get(in[2 * d + 1], c >> 1);
      set(o, d, (c & 1) ? perm(y, x, 0x07060302u) : perm(y, x, 0x05040100u));
    }
    out[c] = o;
  }
}

// 16x16 transpose of bytes.  in[j] holds row j (16 bytes); out[c] receives
// column c.  Built from 4x4 byte transposes of dwords: 8 byte-permutes each.
TX_HD void transpose16x16_b8(const u32x4 *in, u32x4 *out) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {     // dword column of the input = 4 columns
#pragma unroll
    for (int d = 0; d < 4; ++d) {   // group of 4 input rows = output dword d
      uint32_t r0 = get(in[4 * d + 0], q), r1 = get(in[4 * d + 1], q);
      uint32_t r2 = get(in[4 * d + 2], q), r3 = get(in[4 * d + 3], q);
      uint32_t t0 = perm(r1, r0, 0x05010400u); // r0b0 r1b0 r0b1 r1b1
      uint32_t t1 = perm(r1, r0, 0x07030602u); // r0b2 r1b2 r0b3 r1b3
      uint32_t t2 = perm(r3, r2, 0x05010400u);
      uint32_t t3 = perm(r3, r2, 0x07030602u);
      set(out[4 * q + 0], d, perm(t2, t0, 0x05040100u));
      set(out[4 * q + 1], d, perm(t2, t0, 0x07060302u));
      set(out[4 * q + 2], d, perm(t3, t1, 0x05040100u));
      set(out[4 * q + 3], d, perm(t3, t1, 0x07060302u));
    }
  }
}

// fp32 -> bf16 bits, round to nearest even; NaN stays a quiet NaN.
TX_HD uint16_t f32_to_bf16_rne(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u)
    return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

#ifdef __HIPCC__
// Two fp32 -> packed bf16 / fp16 (first in the low half), round to nearest
// even, by the hardware conversion the compiler emits for a cast
// (v_cvt_pk_bf16_f32 on gfx950): one instruction per pair, bit-identical
// to f32_to_bf16_rne / f32_to_f16_rne for every non-NaN input (fp32
// denormals are kept, not flushed).
__device__ __forceinline__ uint32_t pk_bf16_rne(float a, float b) {
  typedef __bf16 bf16x2_t_ __attribute__((ext_vector_type(2)));
  const bf16x2_t_ r = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, r);
}
__device__ __forceinline__ uint32_t pk_f16_rne(float a, float b) {
  typedef _Float16 f16x2_t_ __attribute__((ext_vector_type(2)));
  const f16x2_t_ r = {(_Float16)a, (_Float16)b};
  return __builtin_bit_cast(uint32_t, r);
}
#endif

#ifdef __HIPCC__
// fp32 -> fp16 bits, round to nearest even (IEEE conversion).
__device__ __forceinline__ uint16_t f32_to_f16_rne(float f) {
  _Float16 h = (_Float16)f;
  uint16_t r;
  memcpy(&r, &h, 2);
  return r;
}
#endif

// Byte offset of 16-byte chunk `ch` of LDS row `row` (rows of nch chunks).
// XOR swizzle: 8 consecutive rows reading the same logical chunk land on 8
// different chunks, and rows 8 apart differ too, so both the MFMA operand
// reads (32 consecutive rows, one chunk) and the transposed B writes (rows 8
// apart) spread over all banks.
TX_HD uint32_t lds_off(uint32_t row, uint32_t ch, uint32_t nch) {
  uint32_t swz = (row ^ (row >> 3)) & (nch - 1);
  return row * nch * 16u + ((ch ^ swz) << 4);
}

} // namespace txk
