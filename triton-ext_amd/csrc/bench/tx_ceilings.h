/* Hardware-ceiling kernels timed by bench.py (libtx_ceilings.so).  Not part
 * of the dot path: they measure what one MI355X delivers for a plain HBM
 * read and for the bf16 and 8-bit tiles' MFMA streams alone.  Return 0 on success, 1
 * for bad arguments, 3 if the launch failed. */
#ifndef TRITON_EXT_AMD_TX_CEILINGS_H
#define TRITON_EXT_AMD_TX_CEILINGS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Read `bytes` of `buf` (16-byte aligned) once.  variant 0: 16-byte loads,
 * 8 per thread, a contiguous 32 KiB block per workgroup (bytes % 32 KiB ==
 * 0); 1: the same with 4 loads (16 KiB blocks); 2: direct-to-LDS loads
 * through a per-wave ring on 256 workgroups, as the decode kernel streams B
 * (bytes % 8 MiB == 0).  `sink`: 4 device bytes the kernel almost never
 * writes. */
__attribute__((visibility("default"))) int tx_ceiling_read(const void *buf, size_t bytes,
                                                           int variant, void *sink,
                                                           void *stream);

/* `tiles` workgroups of 4 waves, each running `ksteps` x 64 MFMAs
 * v_mfma_f32_32x32x16_bf16 per wave on operands read once from `seed`
 * (64 x 2048 16-byte values, bf16 data), then one fp32 per thread to
 * `out` [tiles * 256].  FLOPs = tiles * 4 * ksteps * 64 * 32768. */
__attribute__((visibility("default"))) int tx_ceiling_mfma_bf16(const void *seed, int tiles,
                                                                int ksteps, float *out,
                                                                void *stream);

/* tx_ceiling_mfma_bf16 with, per wave w, the wall clock (s_memrealtime,
 * 100 MHz) and the shader clock (s_memtime) before and after its MFMA loop
 * in stamps[4 w .. 4 w + 3]: r0, r1, m0, m1. */
__attribute__((visibility("default"))) int tx_ceiling_mfma_bf16_stamped(const void *seed,
                                                                        int tiles, int ksteps,
                                                                        float *out,
                                                                        uint64_t *stamps,
                                                                        void *stream);

/* Where the stamps of tx_phases_bf16 (and tx_phases_8bit) go: 16 words per
 * wave (tiles_m * tiles_n * 4 waves; 8 for the 8-bit tile), written by
 * every launch, so the last one's remain:
 * [0..4] the wall clock (s_memrealtime, 100 MHz) at entry, step 0 landed, K
 * loop done, epilogue issued, stores acknowledged; [5] XCC_ID << 32 |
 * HW_ID; [6] workgroup; [8..12] the shader clock (s_memtime) at the same
 * five points; with probe_step s in [1, ksteps - 2]: [7] the shader clock
 * after step s - 1's barrier, [13..15] before step s's wait for its loads,
 * after it, after its barrier (probe_step -1: none).  Synchronous. */
__attribute__((visibility("default"))) int tx_phases_bf16_setup(uint64_t *stamps,
                                                                int probe_step);

/* `launches` back-to-back launches of the bf16 256x256 tile kernel (the
 * library's gemm16_w4_kernel, built here with its phase stamps) on
 * C = A . B, all row-major and packed: M = 256 tiles_m, N = 256 tiles_n,
 * K = 64 ksteps, tiles ordered in groups of group_m tile rows. */
__attribute__((visibility("default"))) int tx_phases_bf16(const void *A, const void *B, void *C,
                                                          int tiles_m, int tiles_n, int ksteps,
                                                          int group_m, int launches,
                                                          void *stream);

/* `launches` back-to-back launches of the 8-bit 256x256x128 tile kernel
 * (the library's gemm8_w4_kernel, built here with its phase stamps): kind 0
 * fp8 e4m3 with 128-block scales (sa [M][K/128], sb [K/128][N/128] fp32) and
 * bf16 C, kind 1 int8 with int32 C (no scales), kind 2 MX e4m3 and kind 3
 * MX e2m1 (two per byte) with e8m0 scales per 32 elements (sa [M][K/32],
 * sb [N][K/32] bytes) and fp32 C; all row-major and packed, M = 256
 * tiles_m, N = 256 tiles_n, K = 128 ksteps bytes.  Stamps as for
 * tx_phases_bf16, 8 waves a workgroup, through tx_phases_bf16_setup. */
__attribute__((visibility("default"))) int tx_phases_8bit(int kind, const void *A, const void *B,
                                                          void *C, const void *sa,
                                                          const void *sb, int tiles_m,
                                                          int tiles_n, int ksteps, int group_m,
                                                          int launches, void *stream);

/* tx_ceiling_mfma_fp8 with the stamps of tx_ceiling_mfma_bf16_stamped, 8
 * waves a workgroup. */
__attribute__((visibility("default"))) int tx_ceiling_mfma_fp8_stamped(const void *seed,
                                                                       int tiles, int ksteps,
                                                                       float *out,
                                                                       uint64_t *stamps,
                                                                       void *stream);

/* The 8-bit 256x256x128 tile's operand loads alone: `launches` launches of
 * tiles_m x tiles_n workgroups of 8 waves, each loading its tile's A
 * [256][128] and B [128][256] bytes of every K step into LDS through the
 * tile's own load code and order (one step in flight behind the newest, a
 * barrier a step), no MFMAs, nothing read back.  A [256 tiles_m][128 ksteps]
 * and B [128 ksteps][256 tiles_n] row-major, 8-bit.  0 launched; 1 bad
 * argument; 3 launch error. */
__attribute__((visibility("default"))) int tx_ceiling_operand_stream_8bit(
    const void *A, const void *B, int tiles_m, int tiles_n, int ksteps, int group_m, int launches,
    void *stream);

/* `tiles` workgroups of 8 waves, each running `ksteps` x 32 MFMAs
 * v_mfma_f32_16x16x128_f8f6f4 (e4m3) per wave on operands read once from
 * `seed` (64 x 12 x 64 32-byte values, 32-byte aligned), then one fp32 per
 * thread to `out` [tiles * 512].  FLOPs = tiles * 8 * ksteps * 32 * 65536. */
__attribute__((visibility("default"))) int tx_ceiling_mfma_fp8(const void *seed, int tiles,
                                                               int ksteps, float *out,
                                                               void *stream);

#ifdef __cplusplus
}
#endif

#endif
