// Measured hardware ceilings for bench.py: libtx_ceilings.so.
//
// Not part of the dot path and not a drop-in entry point: two kernels that
// time what one MI355X delivers at the two rooflines the dot is priced
// against, so that the headline fractions can be read beside a ceiling the
// same box measured.
//   * tx_ceiling_read: a plain streaming read of a buffer (every byte once,
//     16-byte non-temporal loads, each workgroup one contiguous block), the
//     best case for an HBM-bound kernel such as the W8A8 decode, which reads
//     its B operand once.
//   * tx_ceiling_mfma_bf16: the bf16 256x256 tile kernel's MFMA work alone
//     (the same grid, waves and v_mfma_f32_32x32x16_bf16 count per wave, on
//     operands held in registers, no LDS and no memory traffic in the loop),
//     the ceiling the power-limited clock leaves for the dot's MFMA stream.
//   * tx_ceiling_mfma_fp8: the same for the 8-bit 256x256x128 tile (8 waves
//     of 8 x 4 blocks of v_mfma_f32_16x16x128_f8f6f4 per K step, e4m3).
//   * tx_phases_bf16 / tx_phases_8bit: the bf16 256x256 tile kernel and the
//     8-bit 256x256x128 tile kernel (fp8 block-scaled, int8 -> int32)
//     themselves, built here with their phase stamps on (s_memrealtime, a
//     100 MHz wall clock, and s_memtime, the shader clock, per wave at
//     entry, step 0 landed, K loop done, epilogue issued, stores
//     acknowledged; optionally around one step's barrier), so that bench.py
//     can say where a launch's time goes.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "tx_ceilings.h"

// Stamp buffer and the step whose barrier is stamped (-1: none), set per
// call of tx_phases_bf16.  A wave's 16 words: [0..4] wall clock at stamps
// 0..4, [5] XCC_ID << 32 | HW_ID, [6] workgroup id, [7] shader clock after
// the barrier of step g_phase_step - 1, [8..12] shader clock at stamps 0..4,
// [13..15] shader clock before step g_phase_step's wait, after it, after
// its barrier.
// __constant__: loop-invariant to the compiler, so the step test in the K
// loop is no reload after every barrier.
__constant__ uint64_t *g_phase_buf;
__constant__ int g_phase_step;

#define TX_PHASE_WORDS(wave)                                                               \
  (g_phase_buf + ((int64_t)blockIdx.x * (blockDim.x >> 6) + (wave)) * 16)
#define TX_PHASE_STAMP(i)                                                                      \
  do {                                                                                         \
    const uint64_t rt_ = __builtin_amdgcn_s_memrealtime();                                     \
    const uint64_t mt_ = __builtin_amdgcn_s_memtime();                                         \
    if ((threadIdx.x & 63) == 0) {                                                             \
      uint64_t *w_ = TX_PHASE_WORDS(threadIdx.x >> 6);                                         \
      w_[i] = rt_;                                                                             \
      w_[8 + (i)] = mt_;                                                                       \
      if ((i) == 0) {                                                                          \
        uint32_t x_, h_;                                                                       \
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x_));                      \
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(h_));                       \
        w_[5] = ((uint64_t)x_ << 32) | h_;                                                     \
        w_[6] = blockIdx.x;                                                                    \
      }                                                                                        \
    }                                                                                          \
  } while (0)
#define TX_PHASE_DRAIN() __builtin_amdgcn_s_waitcnt(0x7 << 4) // vmcnt(0): stores acknowledged
#define TX_PHASE_STEP_BARRIER(kt, barrier)                                                     \
  do {                                                                                         \
    if ((kt) == g_phase_step) {                                                                \
      const uint64_t a_ = __builtin_amdgcn_s_memtime();                                        \
      __builtin_amdgcn_s_waitcnt(0x7 << 4);                                                    \
      const uint64_t b_ = __builtin_amdgcn_s_memtime();                                        \
      __syncthreads();                                                                         \
      const uint64_t c_ = __builtin_amdgcn_s_memtime();                                        \
      if ((threadIdx.x & 63) == 0) {                                                           \
        uint64_t *w_ = TX_PHASE_WORDS(threadIdx.x >> 6);                                       \
        w_[13] = a_;                                                                           \
        w_[14] = b_;                                                                           \
        w_[15] = c_;                                                                           \
      }                                                                                        \
    } else {                                                                                   \
      barrier();                                                                               \
      if ((kt) + 1 == g_phase_step) {                                                          \
        const uint64_t t_ = __builtin_amdgcn_s_memtime();                                      \
        if ((threadIdx.x & 63) == 0)                                                           \
          TX_PHASE_WORDS(threadIdx.x >> 6)[7] = t_;                                            \
      }                                                                                        \
    }                                                                                          \
  } while (0)
#include "backend/mi355x/gemm8_w4.h"

namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

// Read: workgroup b reads bytes [b * 4096 U, (b + 1) * 4096 U): U 16-byte
// loads per thread, all issued before any is used.
template <int U> __global__ void __launch_bounds__(256) read_kernel(const u32x4_t *buf, uint32_t *sink) {
  const u32x4_t *p = buf + (size_t)blockIdx.x * 256 * U + threadIdx.x;
  u32x4_t v[U];
#pragma unroll
  for (int u = 0; u < U; ++u)
    v[u] = __builtin_nontemporal_load(p + u * 256);
  u32x4_t x = v[0];
#pragma unroll
  for (int u = 1; u < U; ++u)
    x ^= v[u];
  // keeps the loads; no thread stores unless the xor hits this value
  if ((x.x ^ x.y ^ x.z ^ x.w) == 0x9e3779b9u)
    *sink = x.x;
}

// Read through LDS the way the decode kernel streams B: one wave per
// workgroup quarter, direct-to-LDS non-temporal 16-byte loads into a ring of
// S slots of 8 KiB, waiting only for the oldest slot.
template <int S> __global__ void __launch_bounds__(256) read_lds_kernel(const uint8_t *buf,
                                                                      int64_t per_wave,
                                                                      uint32_t *sink) {
  __shared__ __attribute__((aligned(1024))) uint8_t ring[4][S][8192];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint8_t *p = buf + ((int64_t)blockIdx.x * 4 + wave) * per_wave;
  const int batches = (int)(per_wave / 8192);
  for (int b = 0; b < batches; ++b) {
    uint8_t *slot = ring[wave][b % S];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      __builtin_amdgcn_global_load_lds(p + (int64_t)b * 8192 + i * 1024 + lane * 16,
                                       (lds_void *)(slot + i * 1024), 16, 0, 2);
    if (b >= S - 1) // at most S - 1 batches of 8 loads in flight beyond this one
      __builtin_amdgcn_s_waitcnt((8 * (S - 1)) & 0xf | (((8 * (S - 1)) >> 4) << 14) |
                                 (0x7 << 4) | (0xf << 8));
  }
  __builtin_amdgcn_s_waitcnt(0);
  if (ring[wave][0][lane] == 0xA5 && ring[wave][S - 1][lane] == 0x5A)
    *sink = lane;
}

// MFMA ceiling: 4 waves per workgroup, 16 accumulators of 32x32 per wave
// (128x128), 4 sub-steps of 16 MFMAs per K step, operands from `seed`
// (different per sub-step and wave) kept in registers.  STAMP: per wave,
// the wall clock and the shader clock before and after the loop into st (a
// separate instantiation: the stamps' registers would otherwise spill).
template <bool STAMP>
__global__ void __launch_bounds__(256, 1) mfma_bf16_kernel(const u32x4_t *seed, int ksteps,
                                                           float *out, uint64_t *st) {
  const int lane = threadIdx.x & 63;
  const u32x4_t *s = seed + ((blockIdx.x * 4 + (threadIdx.x >> 6)) % 64) * 64 * 32 + lane;
  u32x4_t a[4][4], b[4][4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[ks][i] = s[(ks * 8 + i) * 64];
      b[ks][i] = s[(ks * 8 + 4 + i) * 64];
    }
  f32x16_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        acc[i][j][r] = 0.f;
  uint64_t r0 = 0, m0 = 0;
  if constexpr (STAMP) {
    __builtin_amdgcn_s_waitcnt(0);
    r0 = __builtin_amdgcn_s_memrealtime();
    m0 = __builtin_amdgcn_s_memtime();
  }
  for (int kt = 0; kt < ksteps; ++kt) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              __builtin_bit_cast(bf16x8_t, b[ks][j]), __builtin_bit_cast(bf16x8_t, a[ks][i]),
              acc[i][j], 0, 0, 0);
  }
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        t += acc[i][j][r];
  if constexpr (STAMP) {
    const uint64_t r1 = __builtin_amdgcn_s_memrealtime(), m1 = __builtin_amdgcn_s_memtime();
    if (lane == 0) {
      uint64_t *w = st + ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 4;
      w[0] = r0;
      w[1] = r1;
      w[2] = m0;
      w[3] = m1;
    }
  }
  out[(size_t)blockIdx.x * 256 + threadIdx.x] = t;
}

// The bf16 256x256 tile with its phase stamps (the macros above).
__global__ void __launch_bounds__(256, 1) phases_bf16_kernel(txk::GemmArgs p) {
  typedef txk::Gemm16W4<txk::OP_BF16, txk::EPI_BF16, 4, false> G;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * (G::A_BYTES + G::B_BYTES)];
  int tm, tn;
  txk::tile_coords(p, tm, tn);
  G::template run<false>(p, (int64_t)tm * G::BM, (int64_t)tn * G::BN, smem);
}

} // namespace

// fp8 MFMA ceiling: 8 waves per workgroup, 8 x 4 accumulators of 16x16 per
// wave (128x64), one v_mfma_f32_16x16x128_f8f6f4 (e4m3 x e4m3, unit scales)
// per block and K step, operands from `seed` kept in registers.
template <bool STAMP>
__global__ void __launch_bounds__(512, 1) mfma_fp8_kernel(const i32x8_t *seed, int ksteps,
                                                          float *out, uint64_t *st) {
  const int lane = threadIdx.x & 63;
  const i32x8_t *s = seed + ((blockIdx.x * 8 + (threadIdx.x >> 6)) % 64) * 12 * 64 + lane;
  i32x8_t a[8], b[4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
    a[i] = s[i * 64];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    b[j] = s[(8 + j) * 64];
  f32x4_t acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  uint64_t r0 = 0, m0 = 0;
  if constexpr (STAMP) {
    __builtin_amdgcn_s_waitcnt(0);
    r0 = __builtin_amdgcn_s_memrealtime();
    m0 = __builtin_amdgcn_s_memtime();
  }
  for (int kt = 0; kt < ksteps; ++kt) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(b[j], a[i], acc[i][j], 0, 0,
                                                                      0, 0, 0, 0);
  }
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      t += acc[i][j][0] + acc[i][j][1] + acc[i][j][2] + acc[i][j][3];
  if constexpr (STAMP) {
    const uint64_t r1 = __builtin_amdgcn_s_memrealtime(), m1 = __builtin_amdgcn_s_memtime();
    if (lane == 0) {
      uint64_t *w = st + ((int64_t)blockIdx.x * 8 + (threadIdx.x >> 6)) * 4;
      w[0] = r0;
      w[1] = r1;
      w[2] = m0;
      w[3] = m1;
    }
  }
  out[(size_t)blockIdx.x * 512 + threadIdx.x] = t;
}

// The 8-bit tile with its phase stamps: fp8 block-scaled (bf16 C), int8
// with int32 C, or MX (e8m0 per 32) e4m3 or e2m1 with fp32 C.
template <int OP, int EPI, int FA = 0, int FB = 0>
__global__ void __launch_bounds__(512, 1) phases_8bit_kernel(txk::GemmArgs p) {
  typedef txk::Gemm8W4<OP, EPI, FA, FB> G;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * G::STAGE];
  int tm, tn;
  txk::tile_coords(p, tm, tn);
  G::template run<false>(p, (int64_t)tm * G::BM, (int64_t)tn * G::BN, smem);
}

// The 8-bit tile's operand stream alone: each K step's 64 KiB of A and B
// loads (the tile's own lane offsets and tile order) into two LDS stages,
// nothing reading them.  Step kt's loads go out once step kt-1's have landed
// (vmcnt: one step in flight behind the newest, as in the tile), then every
// wave meets at the barrier.  The stage contents are never read, so a stage
// refilled while an older load into it is in flight changes nothing timed.
__global__ void __launch_bounds__(512, 1) operand_stream_8bit_kernel(txk::GemmArgs p) {
  typedef txk::Gemm8W4<txk::OP_I8, txk::EPI_I32> G;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * G::STAGE];
  int tm, tn;
  txk::tile_coords(p, tm, tn);
  const int64_t m0 = (int64_t)tm * G::BM, n0 = (int64_t)tn * G::BN;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t lds0 = txk::lds_addr(smem);
  const txk::i32x4_t ra = txk::make_rsrc(p.A, (uint32_t)((p.M - 1) * p.lda + p.K));
  const txk::i32x4_t rb = txk::make_rsrc(p.B, (uint32_t)((p.K - 1) * p.ldb + p.N));
  const txk::i32x4_t z = {0, 0, 0, 0};
  for (int kt = 0; kt < p.k_main_steps; ++kt) {
    const uint32_t st = lds0 + (kt & 1) * G::STAGE;
    G::template issue_part<false, false, 0>(p, m0, n0, ra, rb, z, z, kt, st, wave, true);
    G::template issue_part<false, false, 1>(p, m0, n0, ra, rb, z, z, kt, st, wave, true);
    G::template issue_part<false, false, 2>(p, m0, n0, ra, rb, z, z, kt, st, wave, true);
    G::template issue_part<false, false, 3>(p, m0, n0, ra, rb, z, z, kt, st, wave, true);
    // 8 loads a wave a step: vmcnt(8) leaves only this step's in flight
    __builtin_amdgcn_s_waitcnt((8 & 15) | (7 << 4) | (15 << 8));
    __syncthreads();
  }
  __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
}

extern "C" int tx_ceiling_read(const void *buf, size_t bytes, int variant, void *sink,
                               void *stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (!buf || !sink || (reinterpret_cast<uintptr_t>(buf) & 15))
    return 1;
  if (variant == 0) { // 8 loads per thread: 32 KiB per workgroup
    if (bytes % (4096 * 8))
      return 1;
    hipLaunchKernelGGL(read_kernel<8>, dim3((unsigned)(bytes / (4096 * 8))), dim3(256), 0, s,
                       static_cast<const u32x4_t *>(buf), static_cast<uint32_t *>(sink));
  } else if (variant == 1) { // 4 loads per thread: 16 KiB per workgroup
    if (bytes % (4096 * 4))
      return 1;
    hipLaunchKernelGGL(read_kernel<4>, dim3((unsigned)(bytes / (4096 * 4))), dim3(256), 0, s,
                       static_cast<const u32x4_t *>(buf), static_cast<uint32_t *>(sink));
  } else if (variant == 2) { // direct-to-LDS ring, 256 workgroups of 4 waves
    const int64_t per_wave = (int64_t)bytes / 1024;
    if (per_wave % 8192 || per_wave <= 0)
      return 1;
    hipLaunchKernelGGL(read_lds_kernel<4>, dim3(256), dim3(256), 0, s,
                       static_cast<const uint8_t *>(buf), per_wave, static_cast<uint32_t *>(sink));
  } else {
    return 1;
  }
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

extern "C" int tx_ceiling_mfma_bf16(const void *seed, int tiles, int ksteps, float *out,
                                    void *stream) {
  if (!seed || !out || tiles <= 0 || ksteps < 0 || (reinterpret_cast<uintptr_t>(seed) & 15))
    return 1;
  hipLaunchKernelGGL(mfma_bf16_kernel<false>, dim3(tiles), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const u32x4_t *>(seed), ksteps,
                     out, nullptr);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

extern "C" int tx_ceiling_mfma_bf16_stamped(const void *seed, int tiles, int ksteps, float *out,
                                            uint64_t *stamps, void *stream) {
  if (!seed || !out || !stamps || tiles <= 0 || ksteps < 0 ||
      (reinterpret_cast<uintptr_t>(seed) & 15))
    return 1;
  hipLaunchKernelGGL(mfma_bf16_kernel<true>, dim3(tiles), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const u32x4_t *>(seed), ksteps,
                     out, stamps);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

extern "C" int tx_phases_bf16_setup(uint64_t *stamps, int probe_step) {
  if (!stamps)
    return 1;
  if (hipMemcpyToSymbol(HIP_SYMBOL(g_phase_buf), &stamps, sizeof(stamps)) != hipSuccess ||
      hipMemcpyToSymbol(HIP_SYMBOL(g_phase_step), &probe_step, sizeof(probe_step)) != hipSuccess ||
      hipDeviceSynchronize() != hipSuccess)
    return 3;
  return 0;
}

extern "C" int tx_phases_bf16(const void *A, const void *B, void *C, int tiles_m, int tiles_n,
                              int ksteps, int group_m, int launches, void *stream) {
  if (!A || !B || !C || tiles_m <= 0 || tiles_n <= 0 || ksteps < 2 || group_m <= 0 ||
      launches <= 0 || (int64_t)tiles_m * tiles_n > 65536 || (int64_t)ksteps * 64 > 65536)
    return 1;
  txk::GemmArgs a{};
  a.A = static_cast<const uint8_t *>(A);
  a.B = static_cast<const uint8_t *>(B);
  a.C = C;
  a.M = (int64_t)tiles_m * 256;
  a.N = (int64_t)tiles_n * 256;
  a.K = (int64_t)ksteps * 64;
  a.lda = a.K;
  a.ldb = a.N;
  a.ldc = a.N;
  a.tiles_m = tiles_m;
  a.tiles_n = tiles_n;
  a.k_main_steps = ksteps;
  a.k_masked_steps = 0;
  a.last_ks = 4;
  a.group_m = group_m < tiles_m ? group_m : tiles_m;
  for (int i = 0; i < launches; ++i)
    hipLaunchKernelGGL(phases_bf16_kernel, dim3(tiles_m * tiles_n), dim3(256), 0,
                       static_cast<hipStream_t>(stream), a);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

extern "C" int tx_ceiling_mfma_fp8(const void *seed, int tiles, int ksteps, float *out,
                                   void *stream) {
  if (!seed || !out || tiles <= 0 || ksteps < 0 || (reinterpret_cast<uintptr_t>(seed) & 31))
    return 1;
  hipLaunchKernelGGL(mfma_fp8_kernel<false>, dim3(tiles), dim3(512), 0,
                     static_cast<hipStream_t>(stream), static_cast<const i32x8_t *>(seed), ksteps,
                     out, nullptr);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

extern "C" int tx_ceiling_mfma_fp8_stamped(const void *seed, int tiles, int ksteps, float *out,
                                           uint64_t *stamps, void *stream) {
  if (!seed || !out || !stamps || tiles <= 0 || ksteps < 0 ||
      (reinterpret_cast<uintptr_t>(seed) & 31))
    return 1;
  hipLaunchKernelGGL(mfma_fp8_kernel<true>, dim3(tiles), dim3(512), 0,
                     static_cast<hipStream_t>(stream), static_cast<const i32x8_t *>(seed), ksteps,
                     out, stamps);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

extern "C" int tx_phases_8bit(int kind, const void *A, const void *B, void *C, const void *sa,
                              const void *sb, int tiles_m, int tiles_n, int ksteps, int group_m,
                              int launches, void *stream) {
  if (!A || !B || !C || kind < 0 || kind > 3 || (kind != 1 && (!sa || !sb)) ||
      tiles_m <= 0 || tiles_n <= 0 || ksteps < 2 || group_m <= 0 || launches <= 0 ||
      (int64_t)tiles_m * tiles_n > 65536 || (int64_t)ksteps * 128 > 65536)
    return 1;
  txk::GemmArgs a{};
  a.A = static_cast<const uint8_t *>(A);
  a.B = static_cast<const uint8_t *>(B);
  a.C = C;
  a.sa = static_cast<const float *>(sa);
  a.sb = static_cast<const float *>(sb);
  a.M = (int64_t)tiles_m * 256;
  a.N = (int64_t)tiles_n * 256;
  a.K = (int64_t)ksteps * 128;
  a.lda = a.K;
  a.ldb = a.N;
  a.ldc = a.N;
  a.tiles_m = tiles_m;
  a.tiles_n = tiles_n;
  a.k_main_steps = ksteps;
  a.k_masked_steps = 0;
  a.last_ks = 1;
  a.group_m = group_m < tiles_m ? group_m : tiles_m;
  a.sa_ld = ksteps;            // sa [M][K / 128]
  a.sb_ld = tiles_n * 2;       // sb [K / 128][N / 128]
  if (kind >= 2)               // MX: e8m0 bytes [M][K / 32], [N][K / 32] (fp4: 256 a step)
    a.sa_ld = ksteps * (kind == 3 ? 8 : 4);
  auto fn = kind == 0   ? phases_8bit_kernel<txk::OP_F8, txk::EPI_BLOCK128_BF16>
            : kind == 1 ? phases_8bit_kernel<txk::OP_I8, txk::EPI_I32>
            : kind == 2 ? phases_8bit_kernel<txk::OP_F8, txk::EPI_MX_F32>
                        : phases_8bit_kernel<txk::OP_F8, txk::EPI_MX_F32, 4, 4>;
  for (int i = 0; i < launches; ++i)
    hipLaunchKernelGGL(fn, dim3(tiles_m * tiles_n), dim3(512), 0,
                       static_cast<hipStream_t>(stream), a);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

extern "C" int tx_ceiling_operand_stream_8bit(const void *A, const void *B, int tiles_m,
                                              int tiles_n, int ksteps, int group_m, int launches,
                                              void *stream) {
  if (!A || !B || tiles_m <= 0 || tiles_n <= 0 || ksteps <= 0 || group_m <= 0 || launches <= 0 ||
      (int64_t)tiles_m * tiles_n > 65536 || (int64_t)ksteps * 128 > 65536)
    return 1;
  txk::GemmArgs a{};
  a.A = static_cast<const uint8_t *>(A);
  a.B = static_cast<const uint8_t *>(B);
  a.M = (int64_t)tiles_m * 256;
  a.N = (int64_t)tiles_n * 256;
  a.K = (int64_t)ksteps * 128;
  a.lda = a.K;
  a.ldb = a.N;
  a.ldc = a.N;
  a.tiles_m = tiles_m;
  a.tiles_n = tiles_n;
  a.k_main_steps = ksteps;
  a.group_m = group_m < tiles_m ? group_m : tiles_m;
  for (int i = 0; i < launches; ++i)
    hipLaunchKernelGGL(operand_stream_8bit_kernel, dim3(tiles_m * tiles_n), dim3(512), 0,
                       static_cast<hipStream_t>(stream), a);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}
