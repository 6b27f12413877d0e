/*
 * oracle/tiled_dot.c -- TEST INFRASTRUCTURE ONLY.
 *
 * CPU restatement of what a Triton tiled-dot kernel computes under the Triton
 * interpreter (TRITON_INTERPRET=1, third-party triton-rocm 3.6.0, cited as
 * T:triton/...).  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the checker; the
 * product path (libmi355x_dot.so) never calls it.
 *
 * The kernel being restated:
 *
 *   pid -> (pid_m, pid_n)                            one program per C tile
 *   acc = zeros([BM, BN], fp32 | int32)
 *   for k0 in range(0, K, BK):
 *       a = tl.load(A[pid_m*BM + i, k0 + k], mask=in-bounds, other=0)
 *       b = tl.load(B[k0 + k, pid_n*BN + j], mask=in-bounds, other=0)
 *       acc = tl.dot(a, b, acc)        (bf16 tiles .to(fp32) first)
 *   tl.store(C_tile, epilogue(acc), mask=in-bounds)
 *
 * Interpreter facts it follows:
 *   - programs run one after another (T:runtime/interpreter.py:1353-1357);
 *     they are independent, so a tile subset can be timed and extrapolated;
 *   - masked loads yield `other`, default 0 (:449-455);
 *   - tl.dot is np.matmul(a, b, dtype=acc.dtype) + acc (:630-637): one fp32
 *     (or int32) partial product per K block, added to the accumulator.  The
 *     partial here sums k in ascending order; BLAS may sum in another order,
 *     so fp results agree to rounding, int32 results exactly;
 *   - fp8 operands are widened exactly to fp16 before the matmul (:633-636),
 *     with the generic converter (:202-263): e4m3 0x7F/0xFF decode as +-480,
 *     not NaN (quantisation with amax/448 scales never produces them); e5m2
 *     is the top byte of an fp16, so its widening is exact, inf and NaN
 *     included.  tl.dot accepts any pair of fp8 types
 *     (T:language/semantic.py:1484-1485);
 *   - bf16 <-> fp32 casts use _convert_float with rounding_mode None
 *     (cast_impl, :461-467): widening is exact and NARROWING TRUNCATES
 *     (round toward zero).  Compiled Triton rounds to nearest even.  Both
 *     are offered (OR_ROUND_RTZ / OR_ROUND_RNE); fp32 -> fp16 uses numpy's
 *     astype, i.e. round to nearest even.
 *
 * Epilogues (the scaled variants restate the task's configs, not a Triton
 * builtin):
 *   plain:      C = cast(acc)
 *   ROWCOL:     C = bf16((float(acc_i32) * sa[m]) * sb[n])
 *   BLOCK128:   BK == 128 and, per K block kb,
 *               acc = acc + (dot_f32(a, b) * sa[m][kb]) * sb[kb][n/128]
 *
 * dot_scaled (oracle_dot_scaled, below) restates tl.dot_scaled with e8m0
 * scales (T:language/semantic.py:1611-1665, T:language/core.py:2064-2101),
 * which the interpreter does not implement.
 *
 * Build: see oracle/Makefile (-ffp-contract=off: no FMA contraction, so the
 * epilogue arithmetic is the plain fp32 sequence written here).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

enum { OR_F32 = 0, OR_F16 = 1, OR_BF16 = 2, OR_I8 = 3, OR_F8E4M3 = 4, OR_I32 = 5,
       OR_F8E5M2 = 6, OR_F4E2M1 = 7 };
enum { OR_SCALE_NONE = 0, OR_SCALE_ROWCOL = 1, OR_SCALE_BLOCK128 = 2 };
enum { OR_ROUND_RTZ = 0, OR_ROUND_RNE = 1, OR_ROUND_INTERP = 2 };

/* ---------------- element codecs ---------------- */

float or_bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

uint16_t or_f32_to_bf16(float f, int mode) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) /* NaN */
    return (uint16_t)((u >> 16) | 0x0040u);
  if (mode == OR_ROUND_RNE)
    u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float or_f16_to_f32(uint16_t h) {
  int s = h >> 15, e = (h >> 10) & 31, m = h & 1023;
  double v;
  if (e == 0)
    v = ldexp((double)m, -24);
  else if (e == 31)
    v = m ? NAN : INFINITY;
  else
    v = ldexp(1.0 + m / 1024.0, e - 15);
  return (float)(s ? -v : v);
}

/* fp32 -> fp16, round to nearest even (IEEE). */
uint16_t or_f32_to_f16(float f) {
  uint16_t s = signbit(f) ? 0x8000u : 0;
  double a = fabs((double)f);
  if (isnan(f))
    return (uint16_t)(s | 0x7e00u);
  if (a >= 65520.0) /* rounds past the largest finite half */
    return (uint16_t)(s | 0x7c00u);
  if (a < ldexp(1.0, -14)) { /* subnormal range: quantum 2^-24 */
    double q = rint(a / ldexp(1.0, -24)); /* half-even under FE_TONEAREST */
    return (uint16_t)(s | (uint16_t)q);   /* q == 1024 is the min normal */
  }
  int e;
  frexp(a, &e); /* a = f * 2^e, f in [0.5, 1) */
  e -= 1;       /* a in [2^e, 2^(e+1)) */
  double q = rint(a / ldexp(1.0, e - 10)); /* 1024..2048 */
  if (q >= 2048.0) {
    q /= 2;
    e += 1;
  }
  if (e > 15)
    return (uint16_t)(s | 0x7c00u);
  return (uint16_t)(s | (uint16_t)((e + 15) << 10) | ((uint16_t)q - 1024));
}

float or_e4m3_to_f32(uint8_t b) {
  int s = b >> 7, e = (b >> 3) & 15, m = b & 7;
  double v = e == 0 ? ldexp((double)m, -9) : ldexp(1.0 + m / 8.0, e - 7);
  return (float)(s ? -v : v);
}

/* fp32 -> e4m3fn, round to nearest even, saturating to +-448. */
uint8_t or_f32_to_e4m3(float f) {
  uint8_t s = signbit(f) ? 0x80u : 0;
  double a = fabs((double)f);
  if (isnan(f))
    return (uint8_t)(s | 0x7fu);
  if (a > 448.0)
    a = 448.0;
  int e;
  if (a < ldexp(1.0, -6)) { /* subnormal: quantum 2^-9 */
    double q = rint(a / ldexp(1.0, -9));
    return (uint8_t)(s | (uint8_t)q); /* q == 8 is the min normal 0x08 */
  }
  frexp(a, &e);
  e -= 1;
  double q = rint(a / ldexp(1.0, e - 3)); /* 8..16 */
  if (q >= 16.0) {
    q /= 2;
    e += 1;
  }
  if (e > 8) /* cannot happen after saturation */
    e = 8, q = 14;
  return (uint8_t)(s | (uint8_t)((e + 7) << 3) | ((uint8_t)q - 8));
}

/* fp32 -> e5m2, round to nearest even (IEEE, as torch's float8_e5m2 and
 * compiled Triton's p.to(tl.float8e5)): bias 15, quantum 2^-16 below 2^-14,
 * |x| >= 61440 (the tie above the largest finite 57344) becomes inf. */
uint8_t or_f32_to_e5m2(float f) {
  uint8_t s = signbit(f) ? 0x80u : 0;
  double a = fabs((double)f);
  if (isnan(f))
    return (uint8_t)(s | 0x7fu);
  if (a >= 61440.0)
    return (uint8_t)(s | 0x7cu);
  if (a < ldexp(1.0, -14)) { /* subnormal: quantum 2^-16 */
    double q = rint(a / ldexp(1.0, -16));
    return (uint8_t)(s | (uint8_t)q); /* q == 4 is the min normal 0x04 */
  }
  int e;
  frexp(a, &e);
  e -= 1;
  double q = rint(a / ldexp(1.0, e - 2)); /* 4..8 */
  if (q >= 8.0) {
    q /= 2;
    e += 1;
  }
  return (uint8_t)(s | (uint8_t)((e + 15) << 2) | ((uint8_t)q - 4));
}

/* fp32 -> e5m2 as the interpreter's generic converter does it with
 * rounding_mode RTNE (T:runtime/interpreter.py:202-263, reached from
 * p.to(tl.float8e5) through create_fp_to_fp, :479-483; the cast picks RTNE
 * for fp downcasts, T:language/semantic.py:807-809).  Its steps:
 *   - a subnormal fp32 input is renormalised: exponent 1 - pos, significand
 *     shifted left by pos (pos = 23 - index of its top set bit); zero keeps
 *     significand 0 with exponent bias_in - bias_out;
 *   - exponent clamped to [0, 31]; significand = top 2 bits + bit 20
 *     (round half up, not to even), and a carry to 4 is ORed into the
 *     exponent field, not added: (1.875..2) * 2^e with e + 15 odd gives
 *     2^e;
 *   - exponent 0 from a normal input (|x| < 2^-14): significand >> shift |
 *     1 << (2 - shift), shift = 113 - exponent; numpy's shifts give 0 for
 *     counts outside [0, bits), so the leading one vanishes for shift > 2;
 *     a subnormal fp32 input keeps its renormalised 2 bits as the code.
 */
uint8_t or_f32_to_e5m2_interp(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint32_t sign = u >> 31;
  const int32_t e_in = (int32_t)((u >> 23) & 0xffu);
  uint32_t sig = u & 0x7fffffu;
  int32_t exp = e_in;
  if (e_in == 0) {
    int pos = 0;
    for (int i = 0; i < 23; ++i)
      if ((sig >> i) & 1u)
        pos = 23 - i;
    exp = sig == 0 ? 127 - 15 : 1 - pos;
    sig = (sig << pos) & 0x7fffffu;
  }
  int32_t eo = exp - 127 + 15;
  eo = eo < 0 ? 0 : (eo > 31 ? 31 : eo);
  uint32_t so = ((sig >> 21) & 3u) + ((sig >> 20) & 1u);
  if (eo == 0 && e_in != 0) {
    const int shift = (1 - 15) - (e_in - 127);
    const uint32_t hi = shift < 32 ? so >> shift : 0u;
    const uint32_t lead = (2 - shift >= 0) ? 1u << (2 - shift) : 0u;
    so = (hi | lead) & 0xffu;
  }
  return (uint8_t)(((sign << 7) | ((uint32_t)eo << 2) | so) & 0xffu);
}

void or_f32_to_e5m2_array(const float *x, uint8_t *y, int64_t n, int mode) {
  for (int64_t i = 0; i < n; ++i)
    y[i] = mode == 2 ? or_f32_to_e5m2_interp(x[i]) : or_f32_to_e5m2(x[i]);
}

void or_f32_to_bf16_array(const float *x, uint16_t *y, int64_t n, int mode) {
  for (int64_t i = 0; i < n; ++i)
    y[i] = or_f32_to_bf16(x[i], mode);
}
void or_bf16_to_f32_array(const uint16_t *x, float *y, int64_t n) {
  for (int64_t i = 0; i < n; ++i)
    y[i] = or_bf16_to_f32(x[i]);
}
void or_f32_to_f16_array(const float *x, uint16_t *y, int64_t n) {
  for (int64_t i = 0; i < n; ++i)
    y[i] = or_f32_to_f16(x[i]);
}
void or_f16_to_f32_array(const uint16_t *x, float *y, int64_t n) {
  for (int64_t i = 0; i < n; ++i)
    y[i] = or_f16_to_f32(x[i]);
}
void or_f32_to_e4m3_array(const float *x, uint8_t *y, int64_t n) {
  for (int64_t i = 0; i < n; ++i)
    y[i] = or_f32_to_e4m3(x[i]);
}
void or_e4m3_to_f32_array(const uint8_t *x, float *y, int64_t n) {
  for (int64_t i = 0; i < n; ++i)
    y[i] = or_e4m3_to_f32(x[i]);
}

/* ---------------- MX element codecs (OCP Microscaling Formats v1.0) ----
 * e4m3fn: bias 7, no inf, S.1111.111 is NaN (the MX path follows the OCP
 *         encoding; the interpreter-facing or_e4m3_to_f32 above keeps the
 *         interpreter's +-480 for that code);
 * e5m2:   bias 15, exponent 31 is inf (mantissa 0) or NaN;
 * e2m1:   bias 1, values +-{0, 0.5, 1, 1.5, 2, 3, 4, 6}, no inf or NaN;
 * e8m0:   2^(s - 127), s = 255 is NaN (s = 0 is 2^-127). */
double or_mx_e4m3_to_f64(uint8_t b) {
  int s = b >> 7, e = (b >> 3) & 15, m = b & 7;
  if (e == 15 && m == 7)
    return NAN;
  double v = e == 0 ? ldexp((double)m, -9) : ldexp(1.0 + m / 8.0, e - 7);
  return s ? -v : v;
}

double or_e5m2_to_f64(uint8_t b) {
  int s = b >> 7, e = (b >> 2) & 31, m = b & 3;
  double v;
  if (e == 31)
    v = m ? NAN : INFINITY;
  else
    v = e == 0 ? ldexp((double)m, -16) : ldexp(1.0 + m / 4.0, e - 15);
  return s ? -v : v;
}

double or_e2m1_to_f64(uint8_t nib) {
  int s = (nib >> 3) & 1, e = (nib >> 1) & 3, m = nib & 1;
  double v = e == 0 ? 0.5 * m : ldexp(1.0 + m / 2.0, e - 1);
  return s ? -v : v;
}

double or_e8m0_to_f64(uint8_t x) { return x == 255 ? NAN : ldexp(1.0, (int)x - 127); }

/* Decode n codes (one per byte; e2m1 in the low nibble) of fmt, or of e8m0
 * for fmt == -1, to double. */
void or_mx_decode_array(const uint8_t *x, double *y, int64_t n, int fmt) {
  for (int64_t i = 0; i < n; ++i) {
    switch (fmt) {
    case OR_F8E4M3: y[i] = or_mx_e4m3_to_f64(x[i]); break;
    case OR_F8E5M2: y[i] = or_e5m2_to_f64(x[i]); break;
    case OR_F4E2M1: y[i] = or_e2m1_to_f64((uint8_t)(x[i] & 15)); break;
    case -1: y[i] = or_e8m0_to_f64(x[i]); break;
    default: y[i] = NAN;
    }
  }
}

/* Element (r, k) of an MX operand stored K-contiguous (A: r = m) or
 * (packed B: r = n, read column-wise).  fp8: one byte; e2m1: the nibble of
 * byte k/2, low nibble for even k. */
static double mx_elem(const uint8_t *base, int fmt, int64_t byte, int k_odd) {
  switch (fmt) {
  case OR_F8E4M3: return or_mx_e4m3_to_f64(base[byte]);
  case OR_F8E5M2: return or_e5m2_to_f64(base[byte]);
  case OR_F4E2M1: return or_e2m1_to_f64((uint8_t)(k_odd ? base[byte] >> 4 : base[byte] & 15));
  default: return NAN;
  }
}

/*
 * tl.dot_scaled(lhs, lhs_scale, fmt_a, rhs, rhs_scale, fmt_b, out_dtype=fp32):
 *   C[m][n] = sum_k (A[m][k] * 2^(sa[m][k/32] - 127)) * (B[k][n] * 2^(sb[n][k/32] - 127))
 * sa is uint8 [M][K/32], sb uint8 [N][K/32] (rhs_scale is indexed by column
 * first, T:language/core.py:2078-2080), K % 32 == 0.  A is [M][K] (e2m1:
 * [M][K/2] bytes, lda in elements), B is [K][N] (e2m1: [K/2][N] bytes,
 * packed along K, ldb = bytes per packed row).  Each term is formed and
 * summed exactly in double (e4m3/e5m2/e2m1 values times powers of two are
 * exact; the sum of 128-term blocks of them is exact in double for the
 * magnitudes tested) and rounded once to fp32: the exact result, against
 * which the hardware's fixed-point group sums are judged by tolerance.
 * c_type OR_BF16 rounds that fp32 value with round_mode.
 * One side may be OR_BF16 (its scale pointer is not read): tl.dot_scaled
 * then upcasts the MX side to bf16 and runs a bf16 dot (T:language/core.py
 * :2072-2076), so each MX element becomes bf16(x * 2^(s - 127)), rounded to
 * nearest even through fp32 (exact except past fp32's range), and the
 * products of bf16 values are summed exactly as above.  Returns 0, or -1
 * for an unsupported combination.
 */
static double upcast_bf16(double v) {
  return or_bf16_to_f32(or_f32_to_bf16((float)v, OR_ROUND_RNE));
}

static int dot_scaled_impl(const void *Av, const void *Bv, void *Cv, const uint8_t *sa,
                           const uint8_t *sb, int64_t M, int64_t N, int64_t K, int64_t lda,
                           int64_t ldb, int64_t ldc, int a_fmt, int b_fmt, int c_type,
                           int round_mode, int nthreads, int nv) {
  const uint8_t *A = (const uint8_t *)Av, *B = (const uint8_t *)Bv;
  uint8_t *C = (uint8_t *)Cv;
  if (M < 0 || N < 0 || K < 0 || K % (nv ? 16 : 32))
    return -1;
  /* e4m3 scales per 16 (nv): e2m1 sides only, both upcast to bf16 */
  const int mixed = a_fmt == OR_BF16 || b_fmt == OR_BF16 || nv;
  if (nv && ((a_fmt != OR_F4E2M1 && a_fmt != OR_BF16) || (b_fmt != OR_F4E2M1 && b_fmt != OR_BF16)))
    return -1;
  const int GS = nv ? 16 : 32; /* K per scale */
  if ((a_fmt != OR_F8E4M3 && a_fmt != OR_F8E5M2 && a_fmt != OR_F4E2M1 && a_fmt != OR_BF16) ||
      (b_fmt != OR_F8E4M3 && b_fmt != OR_F8E5M2 && b_fmt != OR_F4E2M1 && b_fmt != OR_BF16) ||
      (a_fmt == OR_BF16 && b_fmt == OR_BF16))
    return -1;
  if (c_type != OR_F32 && c_type != OR_BF16)
    return -1;
  const int64_t G = K / GS;
#ifdef _OPENMP
  if (nthreads <= 0)
    nthreads = omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
#endif
  for (int64_t m = 0; m < M; ++m) {
    double *arow = (double *)malloc(sizeof(double) * (size_t)(K > 0 ? K : 1));
    if (!arow)
      continue; /* left unwritten; the caller's C stays as it was */
    for (int64_t k = 0; k < K; ++k) {
      if (a_fmt == OR_BF16) {
        arow[k] = or_bf16_to_f32(((const uint16_t *)A)[m * lda + k]);
        continue;
      }
      const int64_t byte = a_fmt == OR_F4E2M1 ? m * (lda / 2) + k / 2 : m * lda + k;
      const uint8_t s = sa[m * G + k / GS];
      arow[k] = mx_elem(A, a_fmt, byte, (int)(k & 1)) *
                (nv ? or_mx_e4m3_to_f64(s) : or_e8m0_to_f64(s));
      if (mixed)
        arow[k] = upcast_bf16(arow[k]);
    }
    for (int64_t n = 0; n < N; ++n) {
      double acc = 0.0;
      for (int64_t k = 0; k < K; ++k) {
        double b;
        if (b_fmt == OR_BF16) {
          b = or_bf16_to_f32(((const uint16_t *)B)[k * ldb + n]);
        } else {
          const int64_t byte = b_fmt == OR_F4E2M1 ? (k / 2) * ldb + n : k * ldb + n;
          const uint8_t s = sb[n * G + k / GS];
          b = mx_elem(B, b_fmt, byte, (int)(k & 1)) *
              (nv ? or_mx_e4m3_to_f64(s) : or_e8m0_to_f64(s));
          if (mixed)
            b = upcast_bf16(b);
        }
        acc += arow[k] * b;
      }
      const float f = (float)acc;
      const int64_t off = m * ldc + n;
      if (c_type == OR_F32) {
        memcpy(C + 4 * off, &f, 4);
      } else {
        uint16_t h = or_f32_to_bf16(f, round_mode);
        memcpy(C + 2 * off, &h, 2);
      }
    }
    free(arow);
  }
  return 0;
}

int oracle_dot_scaled(const void *Av, const void *Bv, void *Cv, const uint8_t *sa,
                      const uint8_t *sb, int64_t M, int64_t N, int64_t K, int64_t lda,
                      int64_t ldb, int64_t ldc, int a_fmt, int b_fmt, int c_type,
                      int round_mode, int nthreads) {
  return dot_scaled_impl(Av, Bv, Cv, sa, sb, M, N, K, lda, ldb, ldc, a_fmt, b_fmt, c_type,
                         round_mode, nthreads, 0);
}

/* The same with e4m3 scales, one per 16 K (tl.dot_scaled's fp8e4nv scale
 * tensors, T:language/semantic.py:1597-1609), K % 16 == 0: sa [M][K/16], sb [N][K/16],
 * each element x * decode_e4m3(s), e2m1 (or bf16) operands, both upcast to
 * bf16 -- exact for e2m1 times e4m3 -- then the products summed as above. */
int oracle_dot_scaled_nv16(const void *Av, const void *Bv, void *Cv, const uint8_t *sa,
                           const uint8_t *sb, int64_t M, int64_t N, int64_t K, int64_t lda,
                           int64_t ldb, int64_t ldc, int a_fmt, int b_fmt, int c_type,
                           int round_mode, int nthreads) {
  return dot_scaled_impl(Av, Bv, Cv, sa, sb, M, N, K, lda, ldb, ldc, a_fmt, b_fmt, c_type,
                         round_mode, nthreads, 1);
}

/* ---------------- fused attention forward ----------------
 * The forward of the fused-attention tutorial as the interpreter runs it
 * (R:pass/LoopSplit/06-fused-attention.py:44-93 _attn_fwd_inner, :181-239
 * _attn_fwd): fp16 q, k, v [Z][H][N][D] packed, one program per (z*H + h,
 * block of BM rows), K/V blocks of BN keys:
 *   m_i = -inf, l_i = 1, acc = 0, qk_scale = fp32(sm_scale * 1.44269504)
 *   qk = q @ k^T                         fp32, d ascending
 *   on-band (start_n >= causal_start):   qk = fl(qk*s) + (m >= n ? 0 : -1e6);
 *                                        m_ij = max(m_i, rowmax qk); qk -= m_ij
 *   off-band:                            m_ij = max(m_i, fl(rowmax(qk)*s));
 *                                        qk = fl(qk*s) - m_ij
 *   p = exp2(qk); l_ij = rowsum p (ascending); alpha = exp2(m_i - m_ij)
 *   l_i = l_i*alpha + l_ij; acc = acc*alpha; acc = (fp16(p) @ v) + acc
 *   m_i = m_ij;  finally M = m_i + log2(l_i), o = fp16(acc / l_i)
 * causal_start = start_m*BM (causal) or N.  dtype OR_F16 (the tutorial's),
 * OR_BF16 or OR_F8E5M2 (the tutorial's fp8 provider, :81-82, :774-779) for
 * q, k, v, p and o; all of them [Z][H][N][D] packed here (the tutorial's fp8
 * v is key-contiguous in memory; the values are the same).  Narrowing:
 * fp16 to nearest even always; bf16 by round_mode RTZ (the interpreter) or
 * RNE (compiled Triton); e5m2 by round_mode RNE (compiled Triton, IEEE) or
 * OR_ROUND_INTERP (the interpreter's converter, or_f32_to_e5m2_interp).
 * fp8 operands of the dots are widened exactly to fp16 first, as the
 * interpreter's tl.dot does (T:runtime/interpreter.py:633-637).  mode (tests only) 0: the
 * tutorial's loop over all keys, split at causal_start; 1: the same loop
 * with every block in the masked form (no split); 2: mode 0 without the
 * blocks wholly past the diagonal.  Returns 0, or -1 on bad arguments.
 */
static float attn_ld(const void *base, int64_t i, int dtype) {
  if (dtype == OR_F8E5M2)
    return or_f16_to_f32((uint16_t)(((const uint8_t *)base)[i] << 8));
  const uint16_t h = ((const uint16_t *)base)[i];
  return dtype == OR_BF16 ? or_bf16_to_f32(h) : or_f16_to_f32(h);
}

/* Store f narrowed to dtype; returns the stored value widened back. */
static float attn_st(void *base, int64_t i, float f, int dtype, int round_mode) {
  if (dtype == OR_F8E5M2) {
    const uint8_t c = round_mode == OR_ROUND_INTERP ? or_f32_to_e5m2_interp(f)
                                                    : or_f32_to_e5m2(f);
    if (base)
      ((uint8_t *)base)[i] = c;
    return or_f16_to_f32((uint16_t)(c << 8));
  }
  const uint16_t h = dtype == OR_BF16 ? or_f32_to_bf16(f, round_mode) : or_f32_to_f16(f);
  if (base)
    ((uint16_t *)base)[i] = h;
  return dtype == OR_BF16 ? or_bf16_to_f32(h) : or_f16_to_f32(h);
}

int oracle_attn_fwd(const void *q, const void *k, const void *v, void *o, float *M, int64_t Z,
                    int64_t H, int64_t N, int D, float sm_scale, int causal, int BM, int BN,
                    int mode, int dtype, int round_mode, int nthreads) {
  if (Z < 0 || H < 0 || N < 0 || D <= 0 || BM <= 0 || BN <= 0 || N % BM || N % BN ||
      (dtype != OR_F16 && dtype != OR_BF16 && dtype != OR_F8E5M2))
    return -1;
#define ATTN_LD(x, i) attn_ld((x), (i), dtype)
  const float qk_scale = sm_scale * 1.44269504f;
  const int64_t programs = Z * H * (N / BM);
  int rc = 0;
#ifdef _OPENMP
  if (nthreads <= 0)
    nthreads = omp_get_max_threads();
#pragma omp parallel num_threads(nthreads)
#endif
  {
    float *qb = (float *)malloc(sizeof(float) * (size_t)BM * D);
    float *acc = (float *)malloc(sizeof(float) * (size_t)BM * D);
    float *qk = (float *)malloc(sizeof(float) * (size_t)BM * BN);
    float *pv = (float *)malloc(sizeof(float) * (size_t)BM * D);
    float *m_i = (float *)malloc(sizeof(float) * (size_t)BM);
    float *l_i = (float *)malloc(sizeof(float) * (size_t)BM);
    if (!qb || !acc || !qk || !pv || !m_i || !l_i) {
#ifdef _OPENMP
#pragma omp atomic write
#endif
      rc = -2;
    } else {
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
      for (int64_t pid = 0; pid < programs; ++pid) {
        const int64_t hz = pid / (N / BM), start_m = pid % (N / BM);
        const int64_t base = hz * N * D, m0 = start_m * BM;
        for (int i = 0; i < BM; ++i) {
          for (int d = 0; d < D; ++d) {
            qb[i * D + d] = ATTN_LD(q, base + (m0 + i) * D + d);
            acc[i * D + d] = 0.f;
          }
          m_i[i] = -INFINITY;
          l_i[i] = 1.0f;
        }
        const int64_t causal_start = causal ? m0 : N;
        for (int64_t n0 = 0; n0 < N; n0 += BN) {
          if (mode == 2 && causal && n0 >= m0 + BM)
            break;
          const int masked = mode == 1 || n0 >= causal_start;
          for (int i = 0; i < BM; ++i)
            for (int j = 0; j < BN; ++j) {
              float t = 0.f;
              for (int d = 0; d < D; ++d)
                t += qb[i * D + d] * ATTN_LD(k, base + (n0 + j) * D + d);
              qk[i * BN + j] = t;
            }
          for (int i = 0; i < BM; ++i) {
            float *r = qk + (size_t)i * BN;
            float m_ij;
            if (masked) {
              float mx = -INFINITY;
              for (int j = 0; j < BN; ++j) {
                float t = r[j] * qk_scale;
                t = t + ((!causal || m0 + i >= n0 + j) ? 0.0f : -1.0e6f);
                r[j] = t;
                if (t > mx)
                  mx = t;
              }
              m_ij = m_i[i] > mx ? m_i[i] : mx;
              for (int j = 0; j < BN; ++j)
                r[j] = r[j] - m_ij;
            } else {
              float mx = -INFINITY;
              for (int j = 0; j < BN; ++j)
                if (r[j] > mx)
                  mx = r[j];
              const float ms = mx * qk_scale;
              m_ij = m_i[i] > ms ? m_i[i] : ms;
              for (int j = 0; j < BN; ++j) {
                const float t = r[j] * qk_scale;
                r[j] = t - m_ij;
              }
            }
            float l_ij = 0.f;
            for (int j = 0; j < BN; ++j) {
              r[j] = exp2f(r[j]);
              l_ij += r[j];
            }
            const float alpha = exp2f(m_i[i] - m_ij);
            l_i[i] = l_i[i] * alpha + l_ij;
            for (int d = 0; d < D; ++d)
              acc[i * D + d] = acc[i * D + d] * alpha;
            for (int j = 0; j < BN; ++j) /* p.to(q's type) */
              r[j] = attn_st(NULL, 0, r[j], dtype, round_mode);
            for (int d = 0; d < D; ++d) {
              float t = 0.f;
              for (int j = 0; j < BN; ++j)
                t += r[j] * ATTN_LD(v, base + (n0 + j) * D + d);
              pv[i * D + d] = t;
            }
            for (int d = 0; d < D; ++d)
              acc[i * D + d] = pv[i * D + d] + acc[i * D + d];
            m_i[i] = m_ij;
          }
        }
        for (int i = 0; i < BM; ++i) {
          M[hz * N + m0 + i] = m_i[i] + log2f(l_i[i]);
          for (int d = 0; d < D; ++d)
            attn_st(o, base + (m0 + i) * D + d, acc[i * D + d] / l_i[i], dtype, round_mode);
        }
      }
    }
    free(qb); free(acc); free(qk); free(pv); free(m_i); free(l_i);
  }
#undef ATTN_LD
  return rc;
}

/* ---------------- the tiled dot ---------------- */

static float load_f(const uint8_t *base, int type, int64_t idx) {
  switch (type) {
  case OR_F32: { float v; memcpy(&v, base + 4 * idx, 4); return v; }
  case OR_F16: { uint16_t h; memcpy(&h, base + 2 * idx, 2); return or_f16_to_f32(h); }
  case OR_BF16: { uint16_t h; memcpy(&h, base + 2 * idx, 2); return or_bf16_to_f32(h); }
  case OR_F8E4M3: return or_e4m3_to_f32(base[idx]);
  case OR_F8E5M2: return or_f16_to_f32((uint16_t)(base[idx] << 8));
  default: return 0.f;
  }
}

static int elt_size(int t) {
  switch (t) {
  case OR_F32: case OR_I32: return 4;
  case OR_F16: case OR_BF16: return 2;
  case OR_I8: case OR_F8E4M3: case OR_F8E5M2: return 1;
  default: return 0;
  }
}

/*
 * Run programs [tile_begin, tile_end) of the tiled dot (program id =
 * pid_m * tiles_n + pid_n; tile_end < 0 means all).  Returns 0, or -1 for an
 * unsupported combination.  Row strides are in elements.
 */
int oracle_tiled_dot(const void *Av, const void *Bv, void *Cv, const float *sa,
                     const float *sb, int64_t M, int64_t N, int64_t K,
                     int64_t lda, int64_t ldb, int64_t ldc, int a_type,
                     int b_type, int c_type, int scale_mode, int round_mode,
                     int BM, int BN, int BK, int64_t tile_begin,
                     int64_t tile_end, int nthreads) {
  const uint8_t *A = (const uint8_t *)Av, *B = (const uint8_t *)Bv;
  uint8_t *C = (uint8_t *)Cv;
  if (BM <= 0 || BN <= 0 || BK <= 0 || M < 0 || N < 0 || K < 0)
    return -1;
  const int fp8_pair = (a_type == OR_F8E4M3 || a_type == OR_F8E5M2) &&
                       (b_type == OR_F8E4M3 || b_type == OR_F8E5M2);
  if ((a_type != b_type && !fp8_pair) || !elt_size(a_type) || !elt_size(c_type))
    return -1;
  const int is_int = a_type == OR_I8;
  if (scale_mode == OR_SCALE_BLOCK128 && BK != 128)
    return -1;
  if (scale_mode == OR_SCALE_ROWCOL && !is_int)
    return -1;
  const int64_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  const int64_t ntiles = tiles_m * tiles_n;
  if (tile_end < 0 || tile_end > ntiles)
    tile_end = ntiles;
  if (tile_begin < 0)
    tile_begin = 0;
  const int64_t kblocks = (K + BK - 1) / BK;
  const int64_t sa_ld = (K + 127) / 128, sb_ld = (N + 127) / 128;
  int rc = 0;
#ifdef _OPENMP
  if (nthreads <= 0)
    nthreads = omp_get_max_threads();
#pragma omp parallel num_threads(nthreads)
#endif
  {
    float *af = (float *)calloc((size_t)BM * BK, sizeof(float));
    float *bf = (float *)calloc((size_t)BK * BN, sizeof(float));
    float *part = (float *)calloc((size_t)BM * BN, sizeof(float));
    float *acc = (float *)calloc((size_t)BM * BN, sizeof(float));
    int32_t *ai = (int32_t *)calloc((size_t)BM * BK, sizeof(int32_t));
    int32_t *bi = (int32_t *)calloc((size_t)BK * BN, sizeof(int32_t));
    uint32_t *iacc = (uint32_t *)calloc((size_t)BM * BN, sizeof(uint32_t));
    uint32_t *ipart = (uint32_t *)calloc((size_t)BM * BN, sizeof(uint32_t));
    if (!af || !bf || !part || !acc || !ai || !bi || !iacc || !ipart) {
#ifdef _OPENMP
#pragma omp atomic write
#endif
      rc = -2;
    } else {
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
      for (int64_t pid = tile_begin; pid < tile_end; ++pid) {
        const int64_t m0 = (pid / tiles_n) * BM, n0 = (pid % tiles_n) * BN;
        memset(acc, 0, sizeof(float) * BM * BN);
        memset(iacc, 0, sizeof(uint32_t) * BM * BN);
        for (int64_t kb = 0; kb < kblocks; ++kb) {
          const int64_t k0 = kb * BK;
          /* masked tile loads, other = 0 */
          for (int i = 0; i < BM; ++i)
            for (int k = 0; k < BK; ++k) {
              const int ok = m0 + i < M && k0 + k < K;
              const int64_t idx = (m0 + i) * lda + k0 + k;
              if (is_int)
                ai[i * BK + k] = ok ? (int32_t)((const int8_t *)A)[idx] : 0;
              else
                af[i * BK + k] = ok ? load_f(A, a_type, idx) : 0.f;
            }
          for (int k = 0; k < BK; ++k)
            for (int j = 0; j < BN; ++j) {
              const int ok = k0 + k < K && n0 + j < N;
              const int64_t idx = (k0 + k) * ldb + n0 + j;
              if (is_int)
                bi[k * BN + j] = ok ? (int32_t)((const int8_t *)B)[idx] : 0;
              else
                bf[k * BN + j] = ok ? load_f(B, b_type, idx) : 0.f;
            }
          /* partial = a @ b, k ascending */
          if (is_int) {
            memset(ipart, 0, sizeof(uint32_t) * BM * BN);
            for (int i = 0; i < BM; ++i)
              for (int k = 0; k < BK; ++k) {
                const uint32_t a = (uint32_t)ai[i * BK + k];
                if (!a)
                  continue;
                uint32_t *pr = ipart + (size_t)i * BN;
                const int32_t *br = bi + (size_t)k * BN;
                for (int j = 0; j < BN; ++j)
                  pr[j] += a * (uint32_t)br[j]; /* int32 wrap, like numpy */
              }
            for (int t = 0; t < BM * BN; ++t)
              iacc[t] = ipart[t] + iacc[t];
          } else {
            memset(part, 0, sizeof(float) * BM * BN);
            for (int i = 0; i < BM; ++i)
              for (int k = 0; k < BK; ++k) {
                const float a = af[i * BK + k];
                float *pr = part + (size_t)i * BN;
                const float *br = bf + (size_t)k * BN;
                for (int j = 0; j < BN; ++j)
                  pr[j] += a * br[j];
              }
            if (scale_mode == OR_SCALE_BLOCK128) {
              for (int i = 0; i < BM; ++i) {
                const float s_a = m0 + i < M ? sa[(m0 + i) * sa_ld + kb] : 0.f;
                for (int j = 0; j < BN; ++j) {
                  const float s_b = n0 + j < N ? sb[kb * sb_ld + (n0 + j) / 128] : 0.f;
                  const float t = (part[i * BN + j] * s_a) * s_b;
                  acc[i * BN + j] = acc[i * BN + j] + t;
                }
              }
            } else {
              for (int t = 0; t < BM * BN; ++t)
                acc[t] = part[t] + acc[t];
            }
          }
        }
        /* epilogue + masked store */
        for (int i = 0; i < BM; ++i) {
          const int64_t m = m0 + i;
          if (m >= M)
            break;
          for (int j = 0; j < BN; ++j) {
            const int64_t n = n0 + j;
            if (n >= N)
              break;
            const int64_t off = m * ldc + n;
            if (is_int) {
              const int32_t v = (int32_t)iacc[i * BN + j];
              if (scale_mode == OR_SCALE_ROWCOL) {
                const float f = ((float)v * sa[m]) * sb[n];
                if (c_type == OR_BF16) {
                  uint16_t h = or_f32_to_bf16(f, round_mode);
                  memcpy(C + 2 * off, &h, 2);
                } else if (c_type == OR_F32) {
                  memcpy(C + 4 * off, &f, 4);
                }
              } else if (c_type == OR_I32) {
                memcpy(C + 4 * off, &v, 4);
              }
            } else {
              const float f = acc[i * BN + j];
              if (c_type == OR_F32) {
                memcpy(C + 4 * off, &f, 4);
              } else if (c_type == OR_BF16) {
                uint16_t h = or_f32_to_bf16(f, round_mode);
                memcpy(C + 2 * off, &h, 2);
              } else if (c_type == OR_F16) {
                uint16_t h = or_f32_to_f16(f);
                memcpy(C + 2 * off, &h, 2);
              }
            }
          }
        }
      }
    }
    free(af); free(bf); free(part); free(acc);
    free(ai); free(bi); free(iacc); free(ipart);
  }
  return rc;
}

/*
 * fp8 block quantisation used by the C5 config: values x (fp32, row-major
 * rows x cols) are split into gr x gc groups; each group's scale is
 * amax / 448 (1 if the group is all zero) and q = e4m3_rne_sat(x / scale).
 * scales is [ceil(rows/gr)][ceil(cols/gc)].
 */
void or_quantize_e4m3_groups(const float *x, int64_t rows, int64_t cols,
                             int gr, int gc, uint8_t *q, float *scales) {
  const int64_t sr = (rows + gr - 1) / gr, sc = (cols + gc - 1) / gc;
  for (int64_t bi = 0; bi < sr; ++bi)
    for (int64_t bj = 0; bj < sc; ++bj) {
      float amax = 0.f;
      for (int64_t i = bi * gr; i < rows && i < (bi + 1) * gr; ++i)
        for (int64_t j = bj * gc; j < cols && j < (bj + 1) * gc; ++j) {
          const float a = fabsf(x[i * cols + j]);
          if (a > amax)
            amax = a;
        }
      const float s = amax > 0.f ? amax / 448.0f : 1.0f;
      scales[bi * sc + bj] = s;
      for (int64_t i = bi * gr; i < rows && i < (bi + 1) * gr; ++i)
        for (int64_t j = bj * gc; j < cols && j < (bj + 1) * gc; ++j)
          q[i * cols + j] = or_f32_to_e4m3(x[i * cols + j] / s);
    }
}
