/* Hardware-ceiling kernels timed by bench.py (libtx_ceilings.so).  Not part
 * of the dot path: they measure what one MI355X delivers for a plain HBM
 * read and for the bf16 and 8-bit tiles' MFMA streams alone.  Return 0 on success, 1
 * for bad arguments, 3 if the launch failed. */
#ifndef TRITON_EXT_AMD_TX_CEILINGS_H
#define TRITON_EXT_AMD_TX_CEILINGS_H

#include <stddef.h>

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
