// mi355x_dot extension: libmi355x_dot.so.
//
// The backend half of the plugin: the "mi355x_dot" pass picks a gfx950 kernel
// and launch shape for a planned dot, and the tx_dot_* C-ABI
// (include/triton_ext/tx_dot.h) validates descriptors, runs the pass pipeline
// (arith_intensity -> loop_split -> mi355x_dot, all through
// tritonAddPluginPass) and launches.  The reference's backend directory is
// empty (R:backend/CMakeLists.txt, 0 bytes); the pipeline shape follows its
// registry (R:infra/pass/TritonExtPassInfra.cpp:19-26).

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>

#include "triton_ext/TritonExtPassInfra.h"
#include "triton_ext/tx_attn.h"
#include "triton_ext/tx_dot.h"
#include "triton_ext/tx_passes.h"

#include "attn_fwd.h"
#include "attn_fwd8.h"
#include "mx_upcast.h"

#include "decode16.h"
#include "decode_f8.h"
#include "decode_i8.h"
#include "decode_rows_i8.h"
#include "gemm16_dma.h"
#include "gemm8_w4.h"
#include "splitk_reduce.h"
#include "gemm8_n224.h"
#include "gemm16_w4.h"
#include "gemm_tile.h"

using namespace txk;

namespace {

thread_local std::string g_last_error;

int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

#define TX_HIP_CHECK(expr)                                                     \
  do {                                                                         \
    hipError_t e_ = (expr);                                                    \
    if (e_ != hipSuccess)                                                      \
      return fail(TX_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(e_));  \
  } while (0)

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------------------
// Kernel table: every (operands, tile, epilogue) the backend instantiates.
// ---------------------------------------------------------------------------

typedef void (*GemmKernelFn)(GemmArgs);

struct GemmConfig {
  int op, bm, bn, bk, wm, wn, epi;
  GemmKernelFn fn;
  int bt;        // B K-major (TX_FLAG_B_KMAJOR)
  int lds_bytes; // dynamic LDS (0 for kernels with static LDS)
  int dma;       // 0: register-staged (gemm_tile.h), 1: direct-to-LDS
                 // staging with 64-bit addresses (gemm16_dma.h), 2: 16-bit
                 // 256x256 tile (gemm16_w4.h), 5: 8-bit 256x256x128 and
                 // 256x224x128 tiles (gemm8_w4.h, gemm8_n224.h); 2 and 5
                 // address A and B through 32-bit buffer offsets
  int fmt;       // MX operand formats: MFMA code of A | code of B << 4
};

#define TX_GEMM(OP, BM, BN, BK, WM, WN, EPI)                                   \
  GemmConfig {                                                                 \
    OP, BM, BN, BK, WM, WN, EPI, gemm_tile_kernel<OP, BM, BN, BK, WM, WN, EPI>,\
        0, GemmTile<OP, BM, BN, BK, WM, WN, EPI>::LDS_BYTES, 0                 \
  }
#define TX_GEMM_DMA_S(OP, BM, BN, BK, WM, WN, ST, EPI)                         \
  GemmConfig {                                                                 \
    OP, BM, BN, BK, WM, WN, EPI,                                               \
        gemm16_dma_kernel<OP, BM, BN, BK, WM, WN, ST, EPI>, 0, 0, 1            \
  }
#define TX_GEMM_DMA(OP, BM, BN, BK, WM, WN, EPI)                               \
  TX_GEMM_DMA_S(OP, BM, BN, BK, WM, WN, 2, EPI)

#define TX_GEMM_W4(OP, EPI)                                                    \
  GemmConfig { OP, 256, 256, 64, 2, 2, EPI, gemm16_w4_kernel<OP, EPI, 4>, 0, 0, 2 }
#define TX_GEMM_W4T(OP, EPI)                                                   \
  GemmConfig { OP, 256, 256, 64, 2, 2, EPI, gemm16_w4_kernel<OP, EPI, 4, true>, 1, 0, 2 }
#define TX_GEMM_8(OP, EPI)                                                     \
  GemmConfig { OP, 256, 256, 128, 2, 4, EPI, gemm8_w4_kernel<OP, EPI>, 0, 0, 5 }
// MX (tl.dot_scaled) tiles: MFMA format codes FA, FB (0 e4m3, 1 e5m2,
// 4 e2m1); BK in elements (128 bytes of K per step).
#define TX_GEMM_MX(FA, FB, BK, EPI)                                            \
  GemmConfig {                                                                 \
    OP_F8, 256, 256, BK, 2, 4, EPI, gemm8_w4_kernel<OP_F8, EPI, FA, FB>, 0, 0, \
        5, (FA) | ((FB) << 4)                                                  \
  }
// Unscaled fp8 with e5m2 operands (MFMA format codes FA, FB; fp32 C).
#define TX_GEMM_8F(FA, FB)                                                     \
  GemmConfig {                                                                 \
    OP_F8, 256, 256, 128, 2, 4, EPI_F32, gemm8_w4_kernel<OP_F8, EPI_F32, FA, FB>, \
        0, 0, 5, (FA) | ((FB) << 4)                                            \
  }
// The same with B K-major (TX_FLAG_B_KMAJOR): every 8-bit epilogue but MX's.
#define TX_GEMM_8T(OP, EPI)                                                    \
  GemmConfig { OP, 256, 256, 128, 2, 4, EPI, gemm8_w4_kernel<OP, EPI, 0, 0, true>, 1, 0, 5 }
#define TX_GEMM_8FT(FA, FB)                                                    \
  GemmConfig {                                                                 \
    OP_F8, 256, 256, 128, 2, 4, EPI_F32, gemm8_w4_kernel<OP_F8, EPI_F32, FA, FB, true>, \
        1, 0, 5, (FA) | ((FB) << 4)                                            \
  }
#define TX_GEMM_8N(OP, EPI)                                                    \
  GemmConfig { OP, 256, 224, 128, 4, 2, EPI, gemm8_n224_kernel<OP, EPI>, 0, 0, 5 }

// Every (operands, tile, epilogue) instantiated; findGemmConfig takes the
// entry that matches a plan exactly.
const GemmConfig kGemmConfigs[] = {
    // bf16 / fp16 operands, 256x256x64 tiles of 4 waves
    TX_GEMM_W4(OP_BF16, EPI_BF16),
    TX_GEMM_W4(OP_BF16, EPI_F32),
    TX_GEMM_W4(OP_F16, EPI_F32),
    TX_GEMM_W4(OP_F16, EPI_F16),
    // the same with B K-major (TX_FLAG_B_KMAJOR)
    TX_GEMM_W4T(OP_BF16, EPI_BF16),
    TX_GEMM_W4T(OP_BF16, EPI_F32),
    TX_GEMM_W4T(OP_F16, EPI_F32),
    TX_GEMM_W4T(OP_F16, EPI_F16),
    // bf16 / fp16 operands, 128x128x64 tiles: direct-to-LDS staging, 64-bit
    // addresses (operands spanning 2 GiB or more); two stages, two
    // workgroups per CU (three or four stages leave one: 32.3 -> 25.6% of
    // peak at bf16 4096^3)
    TX_GEMM_DMA(OP_BF16, 128, 128, 64, 2, 2, EPI_BF16),
    TX_GEMM_DMA(OP_BF16, 128, 128, 64, 2, 2, EPI_F32),
    TX_GEMM_DMA(OP_F16, 128, 128, 64, 2, 2, EPI_F32),
    TX_GEMM_DMA(OP_F16, 128, 128, 64, 2, 2, EPI_F16),
    // 64x64x32 tiles (the reference's BLOCK of config 0): direct-to-LDS
    // staging, three stages (measured at fp16 512^3: 2 / 3 / 4 / 5 stages
    // 8.35 / 7.40 / 7.83 / 8.71 us; register staging 9.05 us)
    TX_GEMM_DMA_S(OP_BF16, 64, 64, 32, 2, 2, 3, EPI_BF16),
    TX_GEMM_DMA_S(OP_BF16, 64, 64, 32, 2, 2, 3, EPI_F32),
    TX_GEMM_DMA_S(OP_F16, 64, 64, 32, 2, 2, 3, EPI_F32),
    TX_GEMM_DMA_S(OP_F16, 64, 64, 32, 2, 2, 3, EPI_F16),
    // int8 / fp8 operands, 256x256x128 tiles of 8 waves (gemm8_w4.h)
    TX_GEMM_8(OP_I8, EPI_I32),
    TX_GEMM_8(OP_I8, EPI_ROWCOL_BF16),
    TX_GEMM_8(OP_F8, EPI_BLOCK128_BF16),
    TX_GEMM_8(OP_F8, EPI_BLOCK128_F32),
    TX_GEMM_8(OP_F8, EPI_F32),
    // fp8 tt.dot with e5m2 on either side (the tutorial's p . v with fp8e5 p)
    TX_GEMM_8F(1, 1),
    TX_GEMM_8F(0, 1),
    TX_GEMM_8F(1, 0),
    // the same with B K-major (q . k^T, or weights kept [out][in])
    TX_GEMM_8T(OP_I8, EPI_I32),
    TX_GEMM_8T(OP_I8, EPI_ROWCOL_BF16),
    TX_GEMM_8T(OP_F8, EPI_BLOCK128_BF16),
    TX_GEMM_8T(OP_F8, EPI_BLOCK128_F32),
    TX_GEMM_8T(OP_F8, EPI_F32),
    TX_GEMM_8FT(1, 1),
    TX_GEMM_8FT(0, 1),
    TX_GEMM_8FT(1, 0),
    // MX: e8m0-scaled fp8 (e4m3 / e5m2 in any mix) and fp4 (gemm8_w4.h)
    TX_GEMM_MX(0, 0, 128, EPI_MX_F32),
    TX_GEMM_MX(0, 0, 128, EPI_MX_BF16),
    TX_GEMM_MX(0, 1, 128, EPI_MX_F32),
    TX_GEMM_MX(0, 1, 128, EPI_MX_BF16),
    TX_GEMM_MX(1, 0, 128, EPI_MX_F32),
    TX_GEMM_MX(1, 0, 128, EPI_MX_BF16),
    TX_GEMM_MX(1, 1, 128, EPI_MX_F32),
    TX_GEMM_MX(1, 1, 128, EPI_MX_BF16),
    TX_GEMM_MX(4, 4, 256, EPI_MX_F32),
    TX_GEMM_MX(4, 4, 256, EPI_MX_BF16),
    // the same with 256x224 tiles (gemm8_n224.h)
    TX_GEMM_8N(OP_I8, EPI_I32),
    TX_GEMM_8N(OP_I8, EPI_ROWCOL_BF16),
    TX_GEMM_8N(OP_F8, EPI_BLOCK128_BF16),
    TX_GEMM_8N(OP_F8, EPI_BLOCK128_F32),
    TX_GEMM_8N(OP_F8, EPI_F32),
    // int8 operands, int32 accumulation, 128x128x128 register-staged tiles
    TX_GEMM(OP_I8, 128, 128, 128, 2, 2, EPI_I32),
    TX_GEMM(OP_I8, 128, 128, 128, 2, 2, EPI_ROWCOL_BF16),
    // fp8 e4m3 operands, fp32 accumulation, 128x128x128 register-staged tiles
    TX_GEMM(OP_F8, 128, 128, 128, 2, 2, EPI_BLOCK128_BF16),
    TX_GEMM(OP_F8, 128, 128, 128, 2, 2, EPI_BLOCK128_F32),
    TX_GEMM(OP_F8, 128, 128, 128, 2, 2, EPI_F32),
};
constexpr int kNumGemmConfigs = sizeof(kGemmConfigs) / sizeof(kGemmConfigs[0]);

typedef void (*DecodeKernelFn)(DecodeArgs);
const DecodeKernelFn kDecodeKernels[4] = {decode_i8_kernel<1>, decode_i8_kernel<2>,
                                           decode_i8_kernel<3>, decode_i8_kernel<4>};
// The row-parallel decode kernel by slice height (64, 128, 256 rows): rings
// of 6, 4 and 3 slots of 24, 32 and 48 KiB (a 128-row batch: B's 16 KiB and
// the slice's A).
// [B K-major][slice of 64, 128, 256 rows]
const DecodeKernelFn kDecodeRowsKernels[2][3] = {
    {decode_rows_i8_kernel<64, 6>, decode_rows_i8_kernel<128, 4>, decode_rows_i8_kernel<256, 3>},
    {decode_rows_i8_kernel<64, 6, true>, decode_rows_i8_kernel<128, 4, true>,
     decode_rows_i8_kernel<256, 3, true>}};
// The 8-bit ring decode kernel: unscaled fp8 by [B K-major][A e4m3 / e5m2]
// [B e4m3 / e5m2][slice of 16, 32, 48, 64 rows], block-scaled (e4m3) by
// [B K-major][slice], int8 with B K-major (int32 C or W8A8) by slice.
typedef void (*DecodeF8KernelFn)(DecodeF8Args);
#define TX_DF8_SLICES(SC, FA, FB, BT, I8)                                                  \
  {decode_f8_kernel<16, SC, FA, FB, BT, I8>, decode_f8_kernel<32, SC, FA, FB, BT, I8>,     \
   decode_f8_kernel<48, SC, FA, FB, BT, I8>, decode_f8_kernel<64, SC, FA, FB, BT, I8>}
const DecodeF8KernelFn kDecodeF8Kernels[2][2][2][4] = {
    {{TX_DF8_SLICES(false, 0, 0, false, false), TX_DF8_SLICES(false, 0, 1, false, false)},
     {TX_DF8_SLICES(false, 1, 0, false, false), TX_DF8_SLICES(false, 1, 1, false, false)}},
    {{TX_DF8_SLICES(false, 0, 0, true, false), TX_DF8_SLICES(false, 0, 1, true, false)},
     {TX_DF8_SLICES(false, 1, 0, true, false), TX_DF8_SLICES(false, 1, 1, true, false)}}};
const DecodeF8KernelFn kDecodeF8ScaledKernels[2][4] = {TX_DF8_SLICES(true, 0, 0, false, false),
                                                       TX_DF8_SLICES(true, 0, 0, true, false)};
const DecodeF8KernelFn kDecodeI8KmajorKernels[4] = TX_DF8_SLICES(false, 0, 0, true, true);
#undef TX_DF8_SLICES
// The 16-bit decode kernel by [B K-major][bf16][slice rows / 16 - 1], slices
// of 16 .. 96 rows.
typedef void (*Decode16KernelFn)(Decode16Args);
#define TX_D16_SLICES(BF, BT)                                                                  \
  {decode16_kernel<16, BF, BT>, decode16_kernel<32, BF, BT>, decode16_kernel<48, BF, BT>,      \
   decode16_kernel<64, BF, BT>, decode16_kernel<80, BF, BT>, decode16_kernel<96, BF, BT>}
const Decode16KernelFn kDecode16Kernels[2][2][kDec16MaxM / 16] = {
    {TX_D16_SLICES(false, false), TX_D16_SLICES(true, false)},
    {TX_D16_SLICES(false, true), TX_D16_SLICES(true, true)}};
#undef TX_D16_SLICES
// The same with strips of 128 columns, slices of 16 .. 80 rows.
#define TX_D16W_SLICES(BF, BT)                                                                 \
  {decode16_kernel<16, BF, BT, 128>, decode16_kernel<32, BF, BT, 128>,                         \
   decode16_kernel<48, BF, BT, 128>, decode16_kernel<64, BF, BT, 128>,                         \
   decode16_kernel<80, BF, BT, 128>}
const Decode16KernelFn kDecode16WideKernels[2][2][kDec16WideMaxM / 16] = {
    {TX_D16W_SLICES(false, false), TX_D16W_SLICES(true, false)},
    {TX_D16W_SLICES(false, true), TX_D16W_SLICES(true, true)}};
#undef TX_D16W_SLICES

// MFMA format code of an MX operand type (-1 if it has none).
int mxFormat(int32_t t) {
  return t == TX_F8E4M3 ? 0 : t == TX_F8E5M2 ? 1 : t == TX_F4E2M1 ? 4 : -1;
}
// Operand format pair of an fp8 / MX descriptor (0 otherwise, and for e4m3
// on both sides).
int fmtOf(const tx_dot_desc &d) {
  const int fa = mxFormat(d.a_type), fb = mxFormat(d.b_type);
  if (fa < 0 || fb < 0)
    return 0;
  return fa | (fb << 4);
}

// tl.dot_scaled with one bf16 operand: the MX operand is upcast to bf16
// (T:language/core.py:2072-2076) and the bf16 tile runs.  1: A is the MX
// operand, 2: B is, 0: not this form.
int mxUpcastSide(const tx_dot_desc &d) {
  if (d.scale_mode == TX_SCALE_NV16) // e4m3 scales: e2m1 sides upcast (3: both)
    return (d.a_type == TX_F4E2M1 ? 1 : 0) | (d.b_type == TX_F4E2M1 ? 2 : 0);
  if (d.scale_mode != TX_SCALE_MX32)
    return 0;
  if (d.a_type == TX_BF16 && mxFormat(d.b_type) >= 0)
    return 2;
  if (d.b_type == TX_BF16 && mxFormat(d.a_type) >= 0)
    return 1;
  return 0;
}

// Workspace of the upcast form: the MX operand as bf16, 256-byte aligned;
// an upcast B's rows hold N rounded up to 16 columns (16-byte aligned rows
// for the bf16 tile, zeros past N).  The upcast starts after the decode
// kernel's counter region (kDecodeCounterBytes), which it never writes, so
// one workspace serves both kernels in any order.
int64_t mxUpcastLdB(const tx_dot_desc &d) { return TX_MX_UPCAST_LD(d.N); }
int64_t mxUpcastOperandBytes(const tx_dot_desc &d) {
  const int side = mxUpcastSide(d);
  const int64_t a = (side & 1) ? (d.M * d.K * 2 + 255) / 256 * 256 : 0;
  const int64_t b = (side & 2) ? (d.K * mxUpcastLdB(d) * 2 + 255) / 256 * 256 : 0;
  return a + b; // A's upcast first, then B's
}
int64_t mxUpcastWorkspace(const tx_dot_desc &d) {
  return mxUpcastSide(d) ? kDecodeCounterBytes + mxUpcastOperandBytes(d) : 0;
}

// Operand kind and epilogue of a descriptor (-1 if unsupported).
void classify(const tx_dot_desc &d, int *op, int *epi) {
  *op = -1;
  *epi = -1;
  if (mxUpcastSide(d)) {
    *op = OP_BF16; // the bf16 tile on the upcast operand
    if (d.c_type == TX_F32)
      *epi = EPI_F32;
    else if (d.c_type == TX_BF16)
      *epi = EPI_BF16;
    return;
  }
  if (d.scale_mode == TX_SCALE_MX32) {
    const int fa = mxFormat(d.a_type), fb = mxFormat(d.b_type);
    if (fa < 0 || fb < 0 || (fa == 4) != (fb == 4))
      return; // fp8 with fp4 would need steps of different byte widths
    *op = OP_F8;
    if (d.c_type == TX_F32)
      *epi = EPI_MX_F32;
    else if (d.c_type == TX_BF16)
      *epi = EPI_MX_BF16;
    return;
  }
  const bool fp8a = d.a_type == TX_F8E4M3 || d.a_type == TX_F8E5M2;
  const bool fp8b = d.b_type == TX_F8E4M3 || d.b_type == TX_F8E5M2;
  if (fp8a && fp8b && (d.a_type == TX_F8E5M2 || d.b_type == TX_F8E5M2)) {
    // tt.dot of fp8 operands with e5m2 on a side ("all combinations of fp8
    // x fp8 are permitted", T:language/semantic.py:1484-1485): fp32 C
    *op = OP_F8;
    if (d.scale_mode == TX_SCALE_NONE && d.c_type == TX_F32)
      *epi = EPI_F32;
    return;
  }
  if (d.a_type != d.b_type)
    return;
  switch (d.a_type) {
  case TX_BF16:
  case TX_F16:
    if (d.scale_mode != TX_SCALE_NONE)
      return;
    *op = d.a_type == TX_BF16 ? OP_BF16 : OP_F16;
    if (d.c_type == TX_F32)
      *epi = EPI_F32;
    else if (d.c_type == TX_BF16 && d.a_type == TX_BF16)
      *epi = EPI_BF16;
    else if (d.c_type == TX_F16 && d.a_type == TX_F16)
      *epi = EPI_F16;
    return;
  case TX_I8:
    *op = OP_I8;
    if (d.scale_mode == TX_SCALE_NONE && d.c_type == TX_I32)
      *epi = EPI_I32;
    else if (d.scale_mode == TX_SCALE_ROWCOL && d.c_type == TX_BF16)
      *epi = EPI_ROWCOL_BF16;
    return;
  case TX_F8E4M3:
    *op = OP_F8;
    if (d.scale_mode == TX_SCALE_BLOCK128 && d.c_type == TX_BF16)
      *epi = EPI_BLOCK128_BF16;
    else if (d.scale_mode == TX_SCALE_BLOCK128 && d.c_type == TX_F32)
      *epi = EPI_BLOCK128_F32;
    else if (d.scale_mode == TX_SCALE_NONE && d.c_type == TX_F32)
      *epi = EPI_F32;
    return;
  default:
    return;
  }
}

int findGemmConfig(int op, int epi, int bm, int bn, int bk, bool bt, int fmt) {
  for (int i = 0; i < kNumGemmConfigs; ++i) {
    const GemmConfig &c = kGemmConfigs[i];
    if (c.op == op && c.epi == epi && c.bm == bm && c.bn == bn && c.bk == bk &&
        c.bt == (int)bt && c.fmt == fmt)
      return i;
  }
  return -1;
}

// Decode row tiling: slices of 16 * MT rows (MT = ceil(M / 16) up to 4), one
// slice up to M = 64 and slices of 64 beyond.  Slices multiply the B bytes a
// workgroup streams (fewer splits), so they are used only once M outgrows one
// wave's accumulators.
int decodeMT(int64_t M) { return M > 64 ? 4 : (int)cdiv(M > 0 ? M : 1, 16); }

// The row-parallel decode kernel (decode_rows_i8.h), named by a block of 64,
// 128 or 256 rows with 128-row K batches (block_k 128): the 4 waves of a
// workgroup split a slice of block_m rows by 128 columns between them and all
// take every K batch of the strip, so a slice streams B once.
bool decodeRows(const tx_dot_desc &d) {
  // past M = 256, 128 x 128 x 128 names the register-staged 8-bit tile
  return d.block_k == kRowsBatchK &&
         (d.block_m == 64 || d.block_m == 256 || (d.block_m == 128 && d.M <= kDecodeMaxM));
}
int decodeSlices(const tx_dot_desc &d) {
  const int64_t M = d.M > 0 ? d.M : 1;
  return (int)cdiv(M, decodeRows(d) ? d.block_m : 16 * decodeMT(M));
}

// Shapes a decode kernel takes: W8A8 (row x column scales, bf16 C) or a
// plain int8 -> int32 dot (no scales, int32 C, optionally accumulating);
// M <= 256 (the row kernel, named by its block, up to 1024), N up to 4096
// strips, and one arrival counter of the fixed region per (slice, strip).
bool decodeEpilogue(const tx_dot_desc &d) {
  return d.a_type == TX_I8 && d.b_type == TX_I8 &&
         ((d.scale_mode == TX_SCALE_ROWCOL && d.c_type == TX_BF16) ||
          (d.scale_mode == TX_SCALE_NONE && d.c_type == TX_I32));
}
bool useDecode(const tx_dot_desc &d) {
  // K-major B: the row kernel only (decode_rows_i8.h's BT form)
  if (!decodeEpilogue(d) || ((d.flags & TX_FLAG_B_KMAJOR) && !decodeRows(d)) ||
      d.N > (int64_t)kDecodeMaxStrips * kDecodeStripN ||
      d.M > (decodeRows(d) ? kDecodeRowsMaxM : kDecodeMaxM))
    return false;
  return (int64_t)decodeSlices(d) * cdiv(d.N, kDecodeStripN) * 4 <= kDecodeCounterBytes;
}

// The decode kernel's tile as the arith_intensity pass names it: a row slice
// (16 MT rows) x a 128-column strip x 64-row K batches.  A caller's explicit
// block other than this runs the tile it names (or is refused).
bool decodeTile(const tx_dot_desc &d) {
  return d.block_n == kDecodeStripN &&
         (decodeRows(d) || (d.block_m == 16 * decodeMT(d.M) && d.block_k == kDecodeBatchK));
}

// Split-K factor for the decode kernel: a power of two (<= kMaxSplit) so
// that slices * strips * ksplit workgroups cover the CUs about once, each
// with at least four 64-row batches per wave.
int decodeSplit(const tx_dot_desc &d) {
  const int64_t strips = cdiv(d.N, kDecodeStripN) * decodeSlices(d);
  const int64_t batches = cdiv(d.K, d.block_k);
  // the K-interleaved kernel deals a split's 64-row batches to its 4 waves;
  // the row kernel's waves each take all of its 128-row batches
  const int64_t min_batches = decodeRows(d) ? 8 : 4 * kDecodeWaves;
  int ks = 1;
  while (ks < (int)kMaxSplit && strips * ks < 256 && batches / (ks * 2) >= min_batches)
    ks *= 2;
  while (ks > 1 && cdiv(batches, ks) * (ks - 1) >= batches)
    ks >>= 1; // every split must own at least one batch
  return ks;
}

int64_t decodeCounterBytes(const tx_dot_desc &) { return kDecodeCounterBytes; }

int64_t decodeWorkspace(const tx_dot_desc &d, int ksplit) {
  if (ksplit <= 1)
    return 0;
  if (decodeRows(d)) // partials in lane order, per slice and strip
    return decodeCounterBytes(d) +
           ksplit * decode_rows_split_bytes(decodeSlices(d), (int)cdiv(d.N, kDecodeStripN),
                                            d.block_m);
  return decodeCounterBytes(d) + (int64_t)ksplit * d.M * ((d.N + 3) & ~3) * 4;
}

// The 16-bit decode kernel (decode16.h): both operands bf16 or both fp16,
// no scales, C in their type or fp32 (accumulating only into fp32, which
// validate() enforces), B row-major or K-major, M <= 96 (one slice), one
// arrival counter of the fixed region per 64-column strip.
int decode16Rows(const tx_dot_desc &d) { return (int)(16 * cdiv(d.M > 0 ? d.M : 1, 16)); }
bool useDecode16(const tx_dot_desc &d) {
  return (d.a_type == TX_BF16 || d.a_type == TX_F16) && d.b_type == d.a_type &&
         d.scale_mode == TX_SCALE_NONE && (d.c_type == d.a_type || d.c_type == TX_F32) &&
         d.M <= kDec16MaxM && cdiv(d.N, kDec16StripN) <= kDec16MaxStrips;
}
// Its tile as the arith_intensity pass names it: the slice (16 ceil(M / 16)
// rows) x a strip of 64 columns (or of 128, for slices up to 80 rows) x
// 128-row K batches.  (No 16-bit GEMM tile has block_k 128.)
bool decode16Tile(const tx_dot_desc &d) {
  return d.block_m == decode16Rows(d) && d.block_k == kDec16BatchK &&
         (d.block_n == kDec16StripN || (d.block_n == 128 && d.block_m <= kDec16WideMaxM));
}
int64_t decode16Strips(const tx_dot_desc &d) { return cdiv(d.N, d.block_n); }
// Split-K factor: the largest power of two (<= kMaxSplit) with strips x
// splits workgroups at most one per CU (one fits a CU's LDS; a second round
// would run behind the first), each split with at least 4 batches of 128 K
// rows, and every split owning one batch at least.
int decode16Split(const tx_dot_desc &d) {
  const int64_t strips = decode16Strips(d);
  const int64_t batches = cdiv(d.K, kDec16BatchK);
  int ks = 1;
  while (ks < (int)kMaxSplit && strips * ks * 2 <= 256 && batches / (ks * 2) >= 4)
    ks *= 2;
  while (ks > 1 && cdiv(batches, ks) * (ks - 1) >= batches)
    ks >>= 1;
  return ks;
}
int64_t decode16Workspace(const tx_dot_desc &d, int ksplit) {
  if (ksplit <= 1)
    return 0;
  return kDecodeCounterBytes +
         ksplit * decode16_split_bytes(decode16Strips(d), decode16Rows(d), (int)d.block_n);
}

// The 8-bit ring decode kernel (decode_f8.h), B row-major or K-major: fp8 x
// fp8 (e4m3 / e5m2 in any mix) with fp32 C; e4m3 x e4m3 with 128-block scales
// and bf16 / fp32 C; with B K-major also int8 -> int32 and W8A8 at M <= 48
// (past it the row kernel's K-major form; row-major int8 runs decode_i8.h);
// M <= 64, one arrival counter per 128-column strip.
bool useDecodeF8(const tx_dot_desc &d) {
  const bool fa = d.a_type == TX_F8E4M3 || d.a_type == TX_F8E5M2;
  const bool fb = d.b_type == TX_F8E4M3 || d.b_type == TX_F8E5M2;
  const bool kmajor = (d.flags & TX_FLAG_B_KMAJOR) != 0;
  if (d.M > kDec8MaxM || cdiv(d.N, kDec8StripN) > kDec16MaxStrips)
    return false;
  if (d.a_type == TX_I8 && d.b_type == TX_I8)
    return kmajor && d.M <= 48 &&
           ((d.scale_mode == TX_SCALE_NONE && d.c_type == TX_I32) ||
            (d.scale_mode == TX_SCALE_ROWCOL && d.c_type == TX_BF16));
  if (!fa || !fb)
    return false;
  if (d.scale_mode == TX_SCALE_NONE)
    return d.c_type == TX_F32;
  return d.scale_mode == TX_SCALE_BLOCK128 && d.a_type == TX_F8E4M3 &&
         d.b_type == TX_F8E4M3 && (d.c_type == TX_BF16 || d.c_type == TX_F32);
}
// Its tile: the slice (16 ceil(M / 16) rows) x a 128-column strip x 128-row
// K batches (no 8-bit GEMM tile is narrower than 128 rows).
bool decodeF8Tile(const tx_dot_desc &d) {
  return d.block_m == decode16Rows(d) && d.block_n == kDec8StripN && d.block_k == kDec8BatchK;
}
int decodeF8Split(const tx_dot_desc &d) { // decode16Split's rule
  const int64_t strips = cdiv(d.N, kDec8StripN);
  const int64_t batches = cdiv(d.K, kDec8BatchK);
  int ks = 1;
  while (ks < (int)kMaxSplit && strips * ks * 2 <= 256 && batches / (ks * 2) >= 4)
    ks *= 2;
  while (ks > 1 && cdiv(batches, ks) * (ks - 1) >= batches)
    ks >>= 1;
  return ks;
}
int64_t decodeF8Workspace(const tx_dot_desc &d, int ksplit) {
  if (ksplit <= 1)
    return 0;
  return kDecodeCounterBytes +
         ksplit * decode_f8_split_bytes(cdiv(d.N, kDec8StripN), decode16Rows(d));
}

// Split-K on the 256x256 tiles (tx_gemm_split_k): every epilogue but MX's
// (and not for a plan that masks every K step).  The tile kernel stores
// range z's 32-bit sums with its fp32 / int32 epilogue (128-block fp8: the
// scaled fp32 one) into the workspace past the decode counters, [split_k][M]
// [ldp] with ldp = N rounded up to 4; splitk_reduce.h adds them and applies
// the dot's own epilogue.
int64_t splitLdp(const tx_dot_desc &d) { return (d.N + 3) & ~3ll; }
int partialEpi(const tx_dot_desc &d, int op) {
  if (op == OP_I8)
    return EPI_I32;
  if (op == OP_F8 && d.scale_mode == TX_SCALE_BLOCK128)
    return EPI_BLOCK128_F32;
  return EPI_F32;
}
// d: the dot the tile runs (for the MX x bf16 upcast, its bf16 dot: bfDot).
int gemmSplit(const tx_dot_desc &d, int op, int64_t tiles) {
  if (d.block_m != 256 || d.block_n != 256 || d.scale_mode == TX_SCALE_MX32 ||
      d.scale_mode == TX_SCALE_NV16 || (d.flags & TX_FLAG_NO_LOOP_SPLIT) ||
      findGemmConfig(op, partialEpi(d, op), d.block_m, d.block_n, d.block_k,
                     (d.flags & TX_FLAG_B_KMAJOR) != 0, fmtOf(d)) < 0)
    return 1;
  return tx_gemm_split_k(tiles, cdiv(d.K, d.block_k));
}
int64_t gemmSplitWorkspace(const tx_dot_desc &d, int split) {
  return split > 1 ? kDecodeCounterBytes + (int64_t)split * d.M * splitLdp(d) * 4 : 0;
}
// The bf16 dot a tl.dot_scaled with an upcast operand runs on the upcast
// operands (the same tile, split-K and epilogue as that bf16 dot).
tx_dot_desc bfDot(const tx_dot_desc &d) {
  tx_dot_desc e = d;
  if (mxUpcastSide(d)) {
    e.a_type = TX_BF16;
    e.b_type = TX_BF16;
    e.scale_mode = TX_SCALE_NONE;
  }
  return e;
}
// Workspace of a tile plan: the upcast operands (after the counter region),
// then the split-K partials (the same offset from the end of the upcast).
int64_t gemmWorkspace(const tx_dot_desc &d, int split) {
  const int64_t up = mxUpcastWorkspace(d);
  const int64_t sk = gemmSplitWorkspace(d, split);
  return up > 0 && sk > 0 ? up + sk - kDecodeCounterBytes : up + sk;
}

// The 32-bit-offset tiles (gemm16_w4.h, gemm8_w4.h, gemm8_n224.h) address A,
// B and the block scales through buffer offsets: each must span less than
// 2^31 bytes (out-of-range chunks, at offset 2^31, read zeros).
int checkSpans32(const tx_dot_desc &d, const GemmConfig &c) {
  if (c.dma != 2 && c.dma != 5)
    return TX_OK;
  tx_dot_desc e = d; // the operands as the tile reads them
  if (mxUpcastSide(d) & 1)
    e.a_type = TX_BF16, e.lda = d.K;
  if (mxUpcastSide(d) & 2)
    e.b_type = TX_BF16, e.ldb = mxUpcastLdB(d);
  int64_t sa = 0, sb = 0;
  tx_dot_operand_spans(&e, &sa, &sb);
  const int64_t kb = cdiv(d.K, 128);
  if (sa >= TX_SPAN32_LIMIT || sb >= TX_SPAN32_LIMIT ||
      (d.scale_mode == TX_SCALE_BLOCK128 &&
       (d.M * kb * 4 >= TX_SPAN32_LIMIT || kb * cdiv(d.N, 128) * 4 >= TX_SPAN32_LIMIT)))
    return fail(TX_ERR_UNSUPPORTED,
                "the %dx%d tile addresses operands through 32-bit offsets: A spans %lld "
                "bytes, B %lld (limit 2^31); a 128x128 tile takes larger operands",
                c.bm, c.bn, (long long)sa, (long long)sb);
  return TX_OK;
}

// The GEMM-tile kernel id of a descriptor of operand kind `op`.
int32_t gemmKernelOf(const tx_dot_desc &d, int op) {
  return op == OP_I8                     ? TX_KERNEL_GEMM_I8
         : mxUpcastSide(d)             ? TX_KERNEL_GEMM_MX_BF16
         : d.scale_mode == TX_SCALE_MX32 ? TX_KERNEL_GEMM_MX
         : op == OP_F8                   ? TX_KERNEL_GEMM_F8
                                         : TX_KERNEL_GEMM_16BIT;
}

// ---------------------------------------------------------------------------
// The "mi355x_dot" pass: kernel choice and launch shape.
// ---------------------------------------------------------------------------
int txMi355xDotRun(tx_dot_plan *plan) {
  const tx_dot_desc &d = plan->desc;
  int op, epi;
  classify(d, &op, &epi);
  if (op < 0 || epi < 0)
    return fail(TX_ERR_UNSUPPORTED,
                "no kernel for a_type=%d b_type=%d c_type=%d scale_mode=%d",
                d.a_type, d.b_type, d.c_type, d.scale_mode);
  if (useDecodeF8(d) && decodeF8Tile(d)) {
    const int ks = decodeF8Split(d);
    plan->kernel = TX_KERNEL_DECODE_F8;
    plan->split_k = ks;
    plan->grid_x = (int32_t)(cdiv(d.N, kDec8StripN) * ks);
    plan->grid_y = plan->grid_z = 1;
    plan->block_threads = kDecodeWaves * 64;
    plan->workspace_bytes = decodeF8Workspace(d, ks);
    plan->passes_run += 1;
    return TX_OK;
  }
  if (useDecode16(d) && decode16Tile(d)) {
    const int ks = decode16Split(d);
    plan->kernel = TX_KERNEL_DECODE_16BIT;
    plan->split_k = ks;
    plan->grid_x = (int32_t)(decode16Strips(d) * ks);
    plan->grid_y = plan->grid_z = 1;
    plan->block_threads = kDecodeWaves * 64;
    plan->workspace_bytes = decode16Workspace(d, ks);
    plan->passes_run += 1;
    return TX_OK;
  }
  if (useDecode(d) && decodeTile(d)) {
    const int ks = decodeSplit(d);
    plan->kernel = TX_KERNEL_DECODE_I8;
    plan->split_k = ks;
    plan->grid_x = (int32_t)(cdiv(d.N, kDecodeStripN) * ks * decodeSlices(d));
    plan->grid_y = plan->grid_z = 1;
    plan->block_threads = kDecodeWaves * 64;
    plan->workspace_bytes = decodeWorkspace(d, ks);
    plan->passes_run += 1;
    return TX_OK;
  }
  // (the upcast forms run the plain bf16 tile: format pair 0)
  const int ci = findGemmConfig(op, epi, d.block_m, d.block_n, d.block_k,
                                (d.flags & TX_FLAG_B_KMAJOR) != 0,
                                mxUpcastSide(d) ? 0 : fmtOf(d));
  if (ci < 0 && (d.flags & TX_FLAG_B_KMAJOR))
    return fail(TX_ERR_UNSUPPORTED,
                "K-major B is implemented on the 256x256 tiles and the decode kernels "
                "(not for MX operands)");
  if (ci < 0)
    return fail(TX_ERR_UNSUPPORTED, "no instantiated tile %dx%dx%d for this dtype",
                d.block_m, d.block_n, d.block_k);
  const GemmConfig &c = kGemmConfigs[ci];
  const bool upcast = mxUpcastSide(d) != 0;
  const int src = checkSpans32(d, c);
  if (src != TX_OK)
    return src;
  if ((int64_t)plan->m_tiles * plan->n_tiles > INT32_MAX)
    return fail(TX_ERR_UNSUPPORTED, "a grid of %lld tiles (above 2^31)",
                (long long)plan->m_tiles * plan->n_tiles);
  // Tile rows per group of the XCD-aware tile order: 4, except 2 on the 8-bit
  // tile once K spans 8192 bytes or more (a sweep of 1..32: mxfp8 8192^3 ran
  // 2365 TFLOP/s at 2 against 1930 at 4; 4096^3, C5 (K = 7168) and mxfp4
  // 8192^3 (K = 4096 bytes) were as fast or faster at 4).
  const int64_t kbytes = d.K * tx_dtype_bits(d.a_type) / 8;
  plan->group_m = c.dma == 5 && kbytes >= 8192 ? 2 : 4;
  plan->kernel = gemmKernelOf(d, op);
  plan->split_k = gemmSplit(bfDot(d), op, (int64_t)plan->m_tiles * plan->n_tiles);
  plan->grid_x = plan->m_tiles * plan->n_tiles;
  plan->grid_y = plan->split_k;
  plan->grid_z = 1;
  plan->block_threads = c.wm * c.wn * 64;
  plan->workspace_bytes = gemmWorkspace(d, plan->split_k);
  plan->passes_run += 1;
  return TX_OK;
}

int validate(const tx_dot_desc *in, tx_dot_desc *d) {
  if (!in)
    return fail(TX_ERR_INVALID, "descriptor is NULL");
  *d = *in;
  if (d->M < 0 || d->N < 0 || d->K < 0)
    return fail(TX_ERR_INVALID, "negative extent M=%lld N=%lld K=%lld",
                (long long)d->M, (long long)d->N, (long long)d->K);
  if (d->M > INT32_MAX || d->N > INT32_MAX || d->K > INT32_MAX)
    return fail(TX_ERR_INVALID, "extent above 2^31-1");
  const int32_t ba = tx_dtype_bits(d->a_type), bb = tx_dtype_bits(d->b_type),
                bc = tx_dtype_bits(d->c_type);
  if (!ba || !bb || !bc || bc < 8)
    return fail(TX_ERR_INVALID, "unknown dtype");
  const bool bt = (d->flags & TX_FLAG_B_KMAJOR) != 0;
  if (d->scale_mode < TX_SCALE_NONE || d->scale_mode > TX_SCALE_NV16)
    return fail(TX_ERR_INVALID, "unknown scale mode %d", d->scale_mode);
  const bool fp4 = ba == 4 || bb == 4;
  if (fp4 && d->scale_mode != TX_SCALE_MX32 && d->scale_mode != TX_SCALE_NV16)
    return fail(TX_ERR_UNSUPPORTED, "e2m1 operands need TX_SCALE_MX32 or TX_SCALE_NV16");
  if (d->scale_mode == TX_SCALE_NV16) {
    const bool ok_a = d->a_type == TX_F4E2M1 || d->a_type == TX_BF16;
    const bool ok_b = d->b_type == TX_F4E2M1 || d->b_type == TX_BF16;
    if (!ok_a || !ok_b || (d->a_type == TX_BF16 && d->b_type == TX_BF16))
      return fail(TX_ERR_UNSUPPORTED, "e4m3 scales per 16 take e2m1 operands (one may be bf16)");
    if (bt)
      return fail(TX_ERR_UNSUPPORTED, "e4m3-scaled operands take B as [K][N]");
    if (d->K % 16)
      return fail(TX_ERR_UNSUPPORTED, "e4m3 scales need K %% 16 == 0 (one scale per 16)");
    if ((d->M > d->N ? d->M : d->N) * (d->K / 16) >= ((int64_t)1 << 31))
      return fail(TX_ERR_UNSUPPORTED, "scale arrays above 2 GiB");
  }
  if (d->lda == 0) d->lda = d->K;
  if (d->ldb == 0) d->ldb = bt ? d->K : d->N;
  if (d->ldc == 0) d->ldc = d->N;
  if (d->lda < d->K || d->ldb < (bt ? d->K : d->N) || d->ldc < d->N)
    return fail(TX_ERR_INVALID, "row stride shorter than the row");
  if (d->flags & ~(TX_FLAG_NO_LOOP_SPLIT | TX_FLAG_B_KMAJOR | TX_FLAG_ACCUMULATE))
    return fail(TX_ERR_INVALID, "unknown flags 0x%x", d->flags);
  if ((d->flags & TX_FLAG_ACCUMULATE) && d->c_type != TX_F32 && d->c_type != TX_I32)
    return fail(TX_ERR_UNSUPPORTED, "accumulating into C needs an fp32 or int32 C");
  // Bytes of a row of A / of B / of C.  e2m1 B is packed along K: a byte
  // row holds N elements of two K rows.
  const int64_t ldb_b = bb == 4 ? d->ldb : d->ldb * bb / 8;
  if ((d->lda * ba) % 128 || ldb_b % 16 || (d->ldc * bc / 8) % 16)
    return fail(TX_ERR_INVALID, "A/B/C row strides must be multiples of 16 bytes");
  // K and N may be any size (tl.load's mask covers every element): the
  // kernels load the 16-byte chunk that crosses K or N whole and zero or drop
  // its elements past the edge.
  if (d->scale_mode == TX_SCALE_MX32) {
    if (d->K % 32)
      return fail(TX_ERR_UNSUPPORTED, "MX scales need K %% 32 == 0 (one e8m0 per 32)");
    if (bt)
      return fail(TX_ERR_UNSUPPORTED, "MX operands take B as [K][N] (no K-major B)");
    if ((d->M > d->N ? d->M : d->N) * (d->K / 32) >= ((int64_t)1 << 31))
      return fail(TX_ERR_UNSUPPORTED, "MX scale arrays above 2 GiB");
  }
  if ((d->block_m < 0) || (d->block_n < 0) || (d->block_k < 0))
    return fail(TX_ERR_INVALID, "negative tile size");
  return TX_OK;
}

} // namespace

// ---------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------

extern "C" TX_API const char *tx_get_last_error(void) {
  return g_last_error.c_str();
}

extern "C" TX_API const char *tx_kernel_name(int32_t kernel) {
  switch (kernel) {
  case TX_KERNEL_GEMM_16BIT: return "gemm_16bit_mfma32x32x16";
  // 8-bit: the 256-wide tiles use the 16x16 MFMAs, the register-staged
  // smaller tiles the 32x32 ones.
  case TX_KERNEL_GEMM_I8: return "gemm_i8_mfma16x16x64|32x32x32";
  // decode: the K-split kernel uses the 16x16 MFMAs, the row-slice kernel the 32x32 ones.
  case TX_KERNEL_DECODE_I8: return "decode_i8_mfma16x16x64|32x32x32";
  case TX_KERNEL_GEMM_F8: return "gemm_f8_mfma16x16x128|32x32x64_f8f6f4";
  case TX_KERNEL_GEMM_MX: return "gemm_mx_mfma_scale16x16x128";
  case TX_KERNEL_GEMM_MX_BF16: return "mx_upcast_bf16+gemm_16bit_mfma32x32x16";
  case TX_KERNEL_DECODE_16BIT: return "decode_16bit_mfma16x16x32";
  case TX_KERNEL_DECODE_F8: return "decode_8bit_mfma16x16x128_f8f6f4|16x16x64_i8";
  default: return "?";
  }
}

extern "C" TX_API int tx_device_available(void) {
  // Per-device answer, cached: hipGetDeviceProperties is too slow to call on
  // every launch.
  // hipGetDevice fails when no device is visible, so it is the only HIP
  // call on a launch.
  static int cached[64];
  static std::once_flag once[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
    return 0;
  std::call_once(once[dev], [dev] {
    hipDeviceProp_t prop;
    cached[dev] = hipGetDeviceProperties(&prop, dev) == hipSuccess &&
                  std::strncmp(prop.gcnArchName, "gfx950", 6) == 0;
  });
  return cached[dev];
}

extern "C" TX_API int tx_dot_plan_create(const tx_dot_desc *desc,
                                         tx_dot_plan *plan) {
  g_last_error.clear();
  if (!plan)
    return fail(TX_ERR_INVALID, "plan is NULL");
  tx_dot_desc d;
  int rc = validate(desc, &d);
  if (rc != TX_OK)
    return rc;
  std::memset(plan, 0, sizeof(*plan));
  plan->desc = d;
  TxPassManager *pm = txPassManagerCreate();
  const char *pipeline[3] = {"arith_intensity", "loop_split", "mi355x_dot"};
  for (const char *name : pipeline)
    if (tritonAddPluginPass(pm, name) != TP_SUCCESS) {
      txPassManagerDestroy(pm);
      return fail(TX_ERR_NO_PASS, "extension pass '%s' is not registered", name);
    }
  rc = txPassManagerRun(pm, plan);
  txPassManagerDestroy(pm);
  if (rc != TX_OK && g_last_error.empty())
    fail(rc, "plan pipeline failed with status %d", rc);
  return rc;
}

namespace {

int launchGemm(const tx_dot_plan &plan, const void *A, const void *B, void *C,
               const void *sa, const void *sb, void *ws, size_t ws_bytes, hipStream_t stream) {
  const tx_dot_desc &d = plan.desc;
  int op, epi;
  classify(d, &op, &epi);
  const int split = plan.split_k > 1 ? plan.split_k : 1;
  // split-K: the tile kernel with the 32-bit partial epilogue, then the reduction
  const int ci = findGemmConfig(op, split > 1 ? partialEpi(d, op) : epi, d.block_m, d.block_n,
                                d.block_k, (d.flags & TX_FLAG_B_KMAJOR) != 0, fmtOf(d));
  if (ci < 0)
    return fail(TX_ERR_UNSUPPORTED, "plan names a tile that is not instantiated");
  const GemmConfig &c = kGemmConfigs[ci];
  if (plan.grid_x != plan.m_tiles * plan.n_tiles || plan.m_tiles <= 0 ||
      plan.n_tiles <= 0 || plan.block_threads != c.wm * c.wn * 64 ||
      plan.grid_y != split)
    return fail(TX_ERR_INVALID, "plan launch shape does not match its tile");
  const int64_t need = gemmSplitWorkspace(d, split);
  if (need > 0 && (!ws || (int64_t)ws_bytes < need))
    return fail(TX_ERR_WORKSPACE, "split-K needs %lld workspace bytes, got %zu", (long long)need,
                ws_bytes);
  if (need > 0 && (reinterpret_cast<uintptr_t>(ws) & 15))
    return fail(TX_ERR_INVALID, "workspace must be 16-byte aligned");
  static std::once_flag attr_once[kNumGemmConfigs];
  hipError_t attr_err = hipSuccess;
  if (c.lds_bytes > 0)
    std::call_once(attr_once[ci], [&] {
      attr_err = hipFuncSetAttribute(reinterpret_cast<const void *>(c.fn),
                                     hipFuncAttributeMaxDynamicSharedMemorySize,
                                     c.lds_bytes);
    });
  TX_HIP_CHECK(attr_err);

  GemmArgs a;
  a.A = static_cast<const uint8_t *>(A);
  a.B = static_cast<const uint8_t *>(B);
  a.C = C;
  a.sa = static_cast<const float *>(sa);
  a.sb = static_cast<const float *>(sb);
  a.M = d.M;
  a.N = d.N;
  a.K = d.K;
  a.lda = d.lda;
  a.ldb = d.ldb;
  a.ldc = d.ldc;
  const bool mx = d.scale_mode == TX_SCALE_MX32;
  if (mx && d.a_type == TX_F4E2M1) {
    // the kernel steps over bytes: K and lda in bytes of A, B's packed rows
    a.K = d.K / 2;
    a.lda = d.lda / 2;
  }
  a.tiles_m = plan.m_tiles;
  a.tiles_n = plan.n_tiles;
  const int64_t masked_k = d.K - plan.k_split;
  a.k_main_steps = plan.k_main_steps;
  a.k_masked_steps = (int32_t)cdiv(masked_k, d.block_k);
  const int total = a.k_main_steps + a.k_masked_steps;
  const int km = op == OP_BF16 || op == OP_F16 ? 16 : op == OP_I8 ? 32 : 64;
  a.last_ks = total > 0 ? (int32_t)cdiv(d.K - (int64_t)(total - 1) * d.block_k, km) : 0;
  if (a.last_ks > d.block_k / km)
    a.last_ks = d.block_k / km;
  const int gm = plan.group_m > 0 ? plan.group_m : 1;
  a.group_m = plan.m_tiles < gm ? plan.m_tiles : gm;
  a.sa_ld = (int32_t)(mx ? d.K / 32 : cdiv(d.K, 128));
  a.sb_ld = (int32_t)cdiv(d.N, 128);
  a.accumulate = (d.flags & TX_FLAG_ACCUMULATE) != 0;
  if (split == 1) {
    hipLaunchKernelGGL(c.fn, dim3(plan.grid_x), dim3(plan.block_threads),
                       c.lds_bytes, stream, a);
    TX_HIP_CHECK(hipGetLastError());
    return TX_OK;
  }
  // Ranges 0 .. split - 2 of split_steps whole K steps each; the last range
  // the rest, with the dot's own peeled tail (the K-loop fields, shifted).
  uint8_t *const part = static_cast<uint8_t *>(ws) + kDecodeCounterBytes;
  const int ksteps = (int)cdiv(d.K, d.block_k);
  a.split_k = split;
  a.split_steps = ksteps / split;
  a.k_main_steps -= (split - 1) * a.split_steps;
  a.C = part;
  a.ldc = splitLdp(d);
  a.accumulate = 0;
  hipLaunchKernelGGL(c.fn, dim3(plan.grid_x, split), dim3(plan.block_threads), c.lds_bytes,
                     stream, a);
  TX_HIP_CHECK(hipGetLastError());
  txk::SplitReduceArgs r;
  r.part = part;
  r.C = C;
  r.sa = static_cast<const float *>(sa);
  r.sb = static_cast<const float *>(sb);
  r.ldc = d.ldc;
  r.ldp = splitLdp(d);
  r.M = (int32_t)d.M;
  r.N = (int32_t)d.N;
  r.split_k = split;
  r.kind = d.c_type == TX_F32   ? txk::SPLIT_F32
           : d.c_type == TX_I32 ? txk::SPLIT_I32
           : d.c_type == TX_F16 ? txk::SPLIT_F16
           : d.scale_mode == TX_SCALE_ROWCOL ? txk::SPLIT_ROWCOL
                                             : txk::SPLIT_BF16;
  r.acc = (d.flags & TX_FLAG_ACCUMULATE) != 0;
  const int64_t quads = d.M * cdiv(d.N, 4);
  if (quads > 0) {
    hipLaunchKernelGGL(txk::splitk_reduce_kernel, dim3((unsigned)cdiv(quads, 256)), dim3(256), 0,
                       stream, r);
    TX_HIP_CHECK(hipGetLastError());
  }
  return TX_OK;
}

// tl.dot_scaled through bf16: upcast the scaled operand(s) -- one side
// against a bf16 operand (MX), or each e2m1 side under e4m3 scales (NV16) --
// into the workspace (A's first, then B's), then the bf16 tile on them, all
// launches on one stream.
int launchMxUpcast(const tx_dot_plan &plan, const void *A, const void *B, void *C,
                   const void *sa, const void *sb, void *ws, size_t ws_bytes,
                   hipStream_t stream) {
  const tx_dot_desc &d = plan.desc;
  const int side = mxUpcastSide(d);
  const bool nv = d.scale_mode == TX_SCALE_NV16;
  const int64_t need = mxUpcastWorkspace(d);
  if (!side)
    return fail(TX_ERR_INVALID, "plan has no operand to upcast");
  if (!ws || (int64_t)ws_bytes < need)
    return fail(TX_ERR_WORKSPACE, "the upcast needs %lld workspace bytes, got %zu",
                (long long)need, ws_bytes);
  if (reinterpret_cast<uintptr_t>(ws) & 15)
    return fail(TX_ERR_INVALID, "workspace must be 16-byte aligned");
  // past the decode counters, which stay untouched
  uint8_t *const up = static_cast<uint8_t *>(ws) + kDecodeCounterBytes;
  uint16_t *wa = reinterpret_cast<uint16_t *>(up);
  uint16_t *wb = reinterpret_cast<uint16_t *>(
      up + ((side & 1) ? (d.M * d.K * 2 + 255) / 256 * 256 : 0));
  typedef void (*UpFn)(txk::UpcastArgs);
  auto upcast = [&](int one) -> int {
    const int fmt = mxFormat(one == 2 ? d.b_type : d.a_type);
    txk::UpcastArgs u;
    u.src = static_cast<const uint8_t *>(one == 2 ? B : A);
    u.scale = static_cast<const uint8_t *>(one == 2 ? sb : sa);
    u.dst = one == 2 ? wb : wa;
    u.ld_dst = one == 2 ? mxUpcastLdB(d) : d.K;
    u.ld_scale = d.K / (nv ? 16 : 32);
    u.fmt = fmt;
    int64_t threads;
    UpFn fn;
    if (one == 2) {
      u.rows = d.K;
      u.cols = d.N;
      u.ld_src = d.ldb; // fp8: bytes per row; e2m1: bytes per packed row
      threads = (d.K / 8) * cdiv(d.N, 16); // 16 columns x 8 K rows per thread
      fn = nv ? txk::mx_upcast_b_kernel<4, true>
              : fmt == 0 ? txk::mx_upcast_b_kernel<0> : fmt == 1 ? txk::mx_upcast_b_kernel<1>
                                                     : txk::mx_upcast_b_kernel<4>;
    } else {
      u.rows = d.M;
      u.cols = d.K;
      u.ld_src = fmt == 4 ? d.lda / 2 : d.lda;
      threads = d.M * (d.K / 16);
      fn = nv ? txk::mx_upcast_a_kernel<4, true>
              : fmt == 0 ? txk::mx_upcast_a_kernel<0> : fmt == 1 ? txk::mx_upcast_a_kernel<1>
                                                     : txk::mx_upcast_a_kernel<4>;
    }
    if (threads > 0) {
      hipLaunchKernelGGL(fn, dim3((unsigned)cdiv(threads, 256)), dim3(256), 0, stream, u);
      TX_HIP_CHECK(hipGetLastError());
    }
    return TX_OK;
  };
  if (side & 1) {
    const int rc = upcast(1);
    if (rc != TX_OK)
      return rc;
  }
  if (side & 2) {
    const int rc = upcast(2);
    if (rc != TX_OK)
      return rc;
  }
  // The bf16 tile over the upcast operand(s).
  tx_dot_plan g = plan;
  g.desc.a_type = TX_BF16;
  g.desc.b_type = TX_BF16;
  g.desc.scale_mode = TX_SCALE_NONE;
  if (side & 2)
    g.desc.ldb = mxUpcastLdB(d);
  if (side & 1)
    g.desc.lda = d.K;
  g.kernel = TX_KERNEL_GEMM_16BIT;
  // split-K partials after the upcast operands (launchGemm skips a counter
  // region's worth from the workspace it is given)
  const int64_t up_bytes = need - kDecodeCounterBytes;
  return launchGemm(g, (side & 1) ? wa : A, (side & 2) ? wb : B, C, nullptr, nullptr,
                    static_cast<uint8_t *>(ws) + up_bytes, ws_bytes - (size_t)up_bytes, stream);
}

int launchDecode(const tx_dot_plan &plan, const void *A, const void *B, void *C,
                 const void *sa, const void *sb, void *ws, size_t ws_bytes,
                 hipStream_t stream) {
  const tx_dot_desc &d = plan.desc;
  const int mt = decodeMT(d.M);
  if (!useDecode(d))
    return fail(TX_ERR_INVALID, "decode plan with M=%lld", (long long)d.M);
  const int slices = decodeSlices(d);
  const int ks = plan.split_k;
  if (ks < 1 || ks > (int)kMaxSplit || (ks & (ks - 1)))
    return fail(TX_ERR_INVALID, "decode split %d is not a power of two <= %u", ks,
                kMaxSplit);
  if (plan.grid_x != cdiv(d.N, kDecodeStripN) * ks * slices ||
      plan.block_threads != kDecodeWaves * 64)
    return fail(TX_ERR_INVALID, "plan launch shape does not match the decode kernel");
  const int64_t need = decodeWorkspace(d, ks);
  if (need > 0 && (!ws || (int64_t)ws_bytes < need))
    return fail(TX_ERR_WORKSPACE, "decode needs %lld workspace bytes, got %zu",
                (long long)need, ws_bytes);
  DecodeArgs a;
  a.A = static_cast<const int8_t *>(A);
  a.B = static_cast<const int8_t *>(B);
  const bool i32 = d.c_type == TX_I32;
  a.C = i32 ? nullptr : static_cast<uint16_t *>(C);
  a.Ci = i32 ? static_cast<int32_t *>(C) : nullptr;
  a.acc_c = i32 && (d.flags & TX_FLAG_ACCUMULATE) != 0;
  a.sa = static_cast<const float *>(sa);
  a.sb = static_cast<const float *>(sb);
  a.M = (int32_t)d.M;
  a.N = (int32_t)d.N;
  a.K = (int32_t)d.K;
  a.lda = d.lda;
  a.ldb = d.ldb;
  a.ldc = d.ldc;
  a.ksplit = ks;
  a.slices = slices;
  const int64_t batches = cdiv(d.K, d.block_k); // the tile's K batch: 64 or 128 rows
  a.batches_per_split = (int32_t)cdiv(batches, ks);
  a.k_main_batches = (int32_t)(plan.k_split / d.block_k);
  const int64_t counters = decodeCounterBytes(d);
  a.counters = static_cast<uint32_t *>(ws);
  a.partials = need > 0 ? reinterpret_cast<int32_t *>(static_cast<uint8_t *>(ws) + counters)
                        : nullptr;
  const DecodeKernelFn fn =
      decodeRows(d) ? kDecodeRowsKernels[(d.flags & TX_FLAG_B_KMAJOR) != 0]
                                        [d.block_m == 64 ? 0 : d.block_m / 128]
                    : kDecodeKernels[mt - 1];
  hipLaunchKernelGGL(fn, dim3(plan.grid_x),
                     dim3(plan.block_threads), 0, stream, a);
  TX_HIP_CHECK(hipGetLastError());
  return TX_OK;
}

int launchDecode16(const tx_dot_plan &plan, const void *A, const void *B, void *C, void *ws,
                   size_t ws_bytes, hipStream_t stream) {
  const tx_dot_desc &d = plan.desc;
  const int ks = plan.split_k;
  const int64_t need = decode16Workspace(d, ks);
  if (need > 0 && (!ws || (int64_t)ws_bytes < need))
    return fail(TX_ERR_WORKSPACE, "decode needs %lld workspace bytes, got %zu",
                (long long)need, ws_bytes);
  Decode16Args a;
  a.A = static_cast<const uint16_t *>(A);
  a.B = static_cast<const uint16_t *>(B);
  a.C = C;
  a.c_f32 = d.c_type == TX_F32;
  a.acc_c = (d.flags & TX_FLAG_ACCUMULATE) != 0;
  a.M = (int32_t)d.M;
  a.N = (int32_t)d.N;
  a.K = (int32_t)d.K;
  a.lda = d.lda;
  a.ldb = d.ldb;
  a.ldc = d.ldc;
  a.ksplit = ks;
  a.batches_per_split = (int32_t)cdiv(cdiv(d.K, kDec16BatchK), ks);
  a.k_main_batches = (int32_t)(plan.k_split / kDec16BatchK);
  a.counters = static_cast<uint32_t *>(ws);
  a.partials = need > 0 ? reinterpret_cast<float *>(static_cast<uint8_t *>(ws) +
                                                    kDecodeCounterBytes)
                        : nullptr;
  const int bt = (d.flags & TX_FLAG_B_KMAJOR) != 0, bf = d.a_type == TX_BF16,
            slice = decode16Rows(d) / 16 - 1;
  const Decode16KernelFn fn = d.block_n == 128 ? kDecode16WideKernels[bt][bf][slice]
                                               : kDecode16Kernels[bt][bf][slice];
  hipLaunchKernelGGL(fn, dim3(plan.grid_x), dim3(plan.block_threads), 0, stream, a);
  TX_HIP_CHECK(hipGetLastError());
  return TX_OK;
}

int launchDecodeF8(const tx_dot_plan &plan, const void *A, const void *B, void *C,
                   const void *sa, const void *sb, void *ws, size_t ws_bytes,
                   hipStream_t stream) {
  const tx_dot_desc &d = plan.desc;
  const int ks = plan.split_k;
  const int64_t need = decodeF8Workspace(d, ks);
  if (need > 0 && (!ws || (int64_t)ws_bytes < need))
    return fail(TX_ERR_WORKSPACE, "decode needs %lld workspace bytes, got %zu",
                (long long)need, ws_bytes);
  const bool scaled = d.scale_mode == TX_SCALE_BLOCK128;
  DecodeF8Args a;
  a.A = static_cast<const uint8_t *>(A);
  a.B = static_cast<const uint8_t *>(B);
  a.C = C;
  a.sa = d.scale_mode == TX_SCALE_NONE ? nullptr : static_cast<const float *>(sa);
  a.sb = d.scale_mode == TX_SCALE_NONE ? nullptr : static_cast<const float *>(sb);
  a.c_f32 = d.c_type == TX_F32;
  a.acc_c = (d.flags & TX_FLAG_ACCUMULATE) != 0;
  a.rowcol = d.scale_mode == TX_SCALE_ROWCOL;
  a.M = (int32_t)d.M;
  a.N = (int32_t)d.N;
  a.K = (int32_t)d.K;
  a.lda = d.lda;
  a.ldb = d.ldb;
  a.ldc = d.ldc;
  a.sa_ld = (int32_t)cdiv(d.K, 128);
  a.sb_ld = (int32_t)cdiv(d.N, 128);
  a.ksplit = ks;
  a.batches_per_split = (int32_t)cdiv(cdiv(d.K, kDec8BatchK), ks);
  a.k_main_batches = (int32_t)(plan.k_split / kDec8BatchK);
  a.counters = static_cast<uint32_t *>(ws);
  a.partials = need > 0 ? reinterpret_cast<float *>(static_cast<uint8_t *>(ws) +
                                                    kDecodeCounterBytes)
                        : nullptr;
  const int si = decode16Rows(d) / 16 - 1;
  const bool kmajor = (d.flags & TX_FLAG_B_KMAJOR) != 0;
  const DecodeF8KernelFn fn =
      d.a_type == TX_I8 ? kDecodeI8KmajorKernels[si]
      : scaled          ? kDecodeF8ScaledKernels[kmajor][si]
                        : kDecodeF8Kernels[kmajor][d.a_type == TX_F8E5M2][d.b_type == TX_F8E5M2][si];
  hipLaunchKernelGGL(fn, dim3(plan.grid_x), dim3(plan.block_threads), 0, stream, a);
  TX_HIP_CHECK(hipGetLastError());
  return TX_OK;
}

} // namespace

// Scratch of tx_dot_launch_noalloc: one array per GPU (each device holds its
// own copy of a __device__ variable), zero when the code object loads.  Host
// code never uses the name as an address: the device address comes from
// hipGetSymbolAddress, once per device.  Layout: the decode kernel's counter
// region first (kDecodeCounterBytes), then its partials; an MX upcast writes
// after the counter region only (as in every workspace), so it never disturbs
// the counters.
__device__ __attribute__((aligned(256))) uint8_t scratch[TX_NOALLOC_SCRATCH_BYTES];
static_assert(kDecodeCounterBytes % 256 == 0, "upcast scratch stays 256-byte aligned");

namespace {

std::mutex g_scratch_mu;
void *g_scratch_ptr[64]; // device address of `scratch`, per device ordinal

// Device address of this GPU's scratch array (the current device).
int scratchOfCurrentDevice(uint8_t **out) {
  int dev = -1;
  TX_HIP_CHECK(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64)
    return fail(TX_ERR_NO_DEVICE, "device ordinal %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    TX_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p)
      return fail(TX_ERR_HIP, "hipGetSymbolAddress(scratch) returned NULL");
    g_scratch_ptr[dev] = p;
  }
  *out = static_cast<uint8_t *>(g_scratch_ptr[dev]);
  return TX_OK;
}

// Checks shared by both launch entry points, then the launch itself.
// noalloc: the workspace is this GPU's scratch array (ws is ignored).
// A plan comes back from the caller at launch.  The fields the kernels trust
// (the loop split, the tile grid, the kernel, its launch shape and workspace)
// must still follow from the plan's descriptor, itself one that validate()
// leaves unchanged, so that a plan edited or built by hand is rejected here,
// before any HIP call, rather than launched with shapes its kernel does not
// assume.  Host arithmetic only: the pass pipeline is not rerun.
int checkPlan(const tx_dot_plan &p) {
  const tx_dot_desc &d = p.desc;
  tx_dot_desc v;
  const int vrc = validate(&d, &v);
  if (vrc != TX_OK)
    return vrc;
  static_assert(sizeof(tx_dot_desc) == 6 * 8 + 8 * 4, "tx_dot_desc has no padding");
  if (std::memcmp(&v, &d, sizeof v) != 0)
    return fail(TX_ERR_INVALID, "the plan's descriptor is not a resolved one (strides left 0)");
  if (d.block_m <= 0 || d.block_n <= 0 || d.block_k <= 0)
    return fail(TX_ERR_INVALID, "the plan has no tile size");
  int64_t ks = 0;
  int32_t km = 0, kt = (int32_t)d.K;
  if (!(d.flags & TX_FLAG_NO_LOOP_SPLIT) && tx_loop_split_k(d.K, d.block_k, &ks, &km, &kt) != TX_OK)
    return fail(TX_ERR_INVALID, "no loop split for K=%lld, BK=%d", (long long)d.K, d.block_k);
  if (p.k_split != ks || p.k_main_steps != km || p.k_tail != kt ||
      p.m_tiles != cdiv(d.M, d.block_m) || p.n_tiles != cdiv(d.N, d.block_n) ||
      p.m_edge != d.M % d.block_m || p.n_edge != d.N % d.block_n || p.grid_z != 1 ||
      (p.grid_y != 1 && p.kernel != TX_KERNEL_GEMM_16BIT && p.kernel != TX_KERNEL_GEMM_I8 &&
       p.kernel != TX_KERNEL_GEMM_F8 && p.kernel != TX_KERNEL_GEMM_MX_BF16))
    // (the tiles' split-K ranges, checked below)
    return fail(TX_ERR_INVALID, "the plan's loop split or tile grid does not follow from its "
                "descriptor");
  int op, epi;
  classify(d, &op, &epi);
  if (op < 0 || epi < 0)
    return fail(TX_ERR_UNSUPPORTED, "no kernel for the plan's operand types");
  if (p.kernel == TX_KERNEL_DECODE_F8) {
    const int sk = p.split_k;
    if (!useDecodeF8(d) || !decodeF8Tile(d) || sk < 1 || sk > (int)kMaxSplit ||
        (sk & (sk - 1)) || p.grid_x != cdiv(d.N, kDec8StripN) * sk ||
        p.block_threads != kDecodeWaves * 64 || p.workspace_bytes != decodeF8Workspace(d, sk))
      return fail(TX_ERR_INVALID, "the plan's decode launch does not follow from its descriptor");
    return TX_OK;
  }
  if (p.kernel == TX_KERNEL_DECODE_16BIT) {
    const int sk = p.split_k;
    if (!useDecode16(d) || !decode16Tile(d) || sk < 1 || sk > (int)kMaxSplit ||
        (sk & (sk - 1)) || p.grid_x != decode16Strips(d) * sk ||
        p.block_threads != kDecodeWaves * 64 || p.workspace_bytes != decode16Workspace(d, sk))
      return fail(TX_ERR_INVALID, "the plan's decode launch does not follow from its descriptor");
    return TX_OK;
  }
  if (p.kernel == TX_KERNEL_DECODE_I8) {
    const int sk = p.split_k;
    if (!useDecode(d) || !decodeTile(d) || sk < 1 || sk > (int)kMaxSplit ||
        (sk & (sk - 1)) || p.grid_x != cdiv(d.N, kDecodeStripN) * sk * decodeSlices(d) ||
        p.block_threads != kDecodeWaves * 64 || p.workspace_bytes != decodeWorkspace(d, sk))
      return fail(TX_ERR_INVALID, "the plan's decode launch does not follow from its descriptor");
    return TX_OK;
  }
  const bool upcast = mxUpcastSide(d) != 0;
  const int ci = findGemmConfig(op, epi, d.block_m, d.block_n, d.block_k,
                                (d.flags & TX_FLAG_B_KMAJOR) != 0, upcast ? 0 : fmtOf(d));
  if (ci < 0)
    return fail(TX_ERR_UNSUPPORTED, "the plan names a tile that is not instantiated");
  const GemmConfig &c = kGemmConfigs[ci];
  const int src = checkSpans32(d, c);
  if (src != TX_OK)
    return src;
  const int split = gemmSplit(bfDot(d), op, (int64_t)p.m_tiles * p.n_tiles);
  if (p.kernel != gemmKernelOf(d, op) || p.split_k != split || p.grid_y != split ||
      p.grid_x != (int64_t)p.m_tiles * p.n_tiles || p.block_threads != c.wm * c.wn * 64 ||
      p.workspace_bytes != gemmWorkspace(d, split))
    return fail(TX_ERR_INVALID, "the plan's kernel or launch shape does not follow from its "
                "descriptor");
  return TX_OK;
}

int launchPlanned(const tx_dot_plan *plan, const void *A, const void *B, void *C,
                  const void *scale_a, const void *scale_b, void *workspace,
                  size_t workspace_bytes, void *stream, bool noalloc) {
  if (!plan)
    return fail(TX_ERR_INVALID, "plan is NULL");
  const tx_dot_desc &d = plan->desc;
  if (d.M == 0 || d.N == 0)
    return TX_OK; // empty output
  if (!C || (d.K > 0 && (!A || !B)))
    return fail(TX_ERR_INVALID, "NULL operand pointer");
  if ((reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(B) |
       reinterpret_cast<uintptr_t>(C)) & 15)
    return fail(TX_ERR_INVALID, "A, B and C must be 16-byte aligned");
  // MX x bf16 (dot_scaled with one bf16 operand): only the MX side is scaled
  const int up = mxUpcastSide(d);
  const bool need_sa = d.scale_mode != TX_SCALE_NONE && up != 2;
  const bool need_sb = d.scale_mode != TX_SCALE_NONE && up != 1;
  if ((need_sa && !scale_a) || (need_sb && !scale_b))
    return fail(TX_ERR_INVALID, "scaled dot needs scale_a and scale_b");
  if (((need_sa ? reinterpret_cast<uintptr_t>(scale_a) : 0) |
       (need_sb ? reinterpret_cast<uintptr_t>(scale_b) : 0)) & 3)
    return fail(TX_ERR_INVALID, "scale arrays must be 4-byte aligned");
  const int prc = checkPlan(*plan);
  if (prc != TX_OK)
    return prc;
  // No allocation: a split-K tile plan whose partials do not fit the scratch
  // runs unsplit (the same dot, one K range a tile).
  tx_dot_plan unsplit;
  if (noalloc && plan->split_k > 1 && plan->grid_y == plan->split_k &&
      plan->workspace_bytes > (int64_t)TX_NOALLOC_SCRATCH_BYTES &&
      (plan->kernel == TX_KERNEL_GEMM_16BIT || plan->kernel == TX_KERNEL_GEMM_I8 ||
       plan->kernel == TX_KERNEL_GEMM_F8 || plan->kernel == TX_KERNEL_GEMM_MX_BF16)) {
    unsplit = *plan;
    unsplit.split_k = 1;
    unsplit.grid_y = 1;
    unsplit.workspace_bytes = gemmWorkspace(plan->desc, 1);
    plan = &unsplit;
  }
  if (noalloc && (plan->workspace_bytes < 0 ||
                  plan->workspace_bytes > (int64_t)TX_NOALLOC_SCRATCH_BYTES))
    return fail(TX_ERR_WORKSPACE,
                "the plan needs %lld bytes of workspace; the no-allocation scratch holds %lld",
                (long long)plan->workspace_bytes, (long long)TX_NOALLOC_SCRATCH_BYTES);
  if (!tx_device_available())
    return fail(TX_ERR_NO_DEVICE, "no gfx950 device visible");
  if (noalloc && plan->workspace_bytes > 0) {
    uint8_t *base = nullptr;
    const int rc = scratchOfCurrentDevice(&base);
    if (rc != TX_OK)
      return rc;
    workspace = base;
    workspace_bytes = TX_NOALLOC_SCRATCH_BYTES;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (plan->kernel) {
  case TX_KERNEL_GEMM_16BIT:
  case TX_KERNEL_GEMM_I8:
  case TX_KERNEL_GEMM_F8:
  case TX_KERNEL_GEMM_MX:
    return launchGemm(*plan, A, B, C, scale_a, scale_b, workspace, workspace_bytes, s);
  case TX_KERNEL_DECODE_I8:
    return launchDecode(*plan, A, B, C, scale_a, scale_b, workspace,
                        workspace_bytes, s);
  case TX_KERNEL_DECODE_16BIT:
    return launchDecode16(*plan, A, B, C, workspace, workspace_bytes, s);
  case TX_KERNEL_DECODE_F8:
    return launchDecodeF8(*plan, A, B, C, scale_a, scale_b, workspace, workspace_bytes, s);
  case TX_KERNEL_GEMM_MX_BF16:
    return launchMxUpcast(*plan, A, B, C, scale_a, scale_b, workspace, workspace_bytes, s);
  default:
    return fail(TX_ERR_INVALID, "plan has no kernel (kernel=%d)", plan->kernel);
  }
}

} // namespace

extern "C" TX_API int tx_dot_launch(const tx_dot_plan *plan, const void *A,
                                    const void *B, void *C,
                                    const void *scale_a, const void *scale_b,
                                    void *workspace, size_t workspace_bytes,
                                    void *stream) {
  g_last_error.clear();
  return launchPlanned(plan, A, B, C, scale_a, scale_b, workspace, workspace_bytes, stream,
                       false);
}

extern "C" TX_API int tx_dot_launch_noalloc(const tx_dot_plan *plan, const void *A,
                                            const void *B, void *C, const void *scale_a,
                                            const void *scale_b, void *stream) {
  g_last_error.clear();
  return launchPlanned(plan, A, B, C, scale_a, scale_b, nullptr, 0, stream, true);
}

// ---------------------------------------------------------------------------
// Fused attention forward (tx_attn.h)
// ---------------------------------------------------------------------------

namespace {

// Packed defaults and checks of one tensor's (batch, head, row) strides.
// key_major: e5m2 v, stored [HEAD_DIM][N_CTX] per head (sm = dim stride).
int attnStrides(const tx_attn_desc &d, int64_t &sz, int64_t &sh, int64_t &sm,
                const char *name, bool key_major) {
  const int64_t esz = d.dtype == TX_F8E5M2 ? 1 : 2, quantum = 16 / esz;
  const int64_t rows = key_major ? d.head_dim : d.N_CTX, len = key_major ? d.N_CTX : d.head_dim;
  if (sm == 0) sm = len;
  if (sh == 0) sh = rows * sm;
  if (sz == 0) sz = d.H * sh;
  if (sm < len || sh < 0 || sz < 0 || sm % quantum || sh % quantum || sz % quantum)
    return fail(TX_ERR_INVALID, "%s strides (%lld, %lld, %lld): rows of %s elements, "
                "multiples of 16 bytes", name, (long long)sz, (long long)sh, (long long)sm,
                key_major ? "N_CTX" : "head_dim");
  if (((rows - 1) * sm + len) * esz >= ((int64_t)1 << 31))
    return fail(TX_ERR_UNSUPPORTED, "%s: one head spans 2 GiB or more", name);
  return TX_OK;
}

} // namespace

extern "C" TX_API int tx_attn_fwd_plan(const tx_attn_desc *desc, tx_attn_plan *plan) {
  g_last_error.clear();
  if (!desc || !plan)
    return fail(TX_ERR_INVALID, "descriptor or plan is NULL");
  tx_attn_desc d = *desc;
  if (d.Z < 0 || d.H < 0 || d.N_CTX < 0)
    return fail(TX_ERR_INVALID, "negative extent Z=%lld H=%lld N_CTX=%lld", (long long)d.Z,
                (long long)d.H, (long long)d.N_CTX);
  if (d.causal != 0 && d.causal != 1)
    return fail(TX_ERR_INVALID, "causal must be 0 or 1");
  if (!(d.sm_scale == d.sm_scale))
    return fail(TX_ERR_INVALID, "sm_scale is NaN");
  if (d.dtype != TX_F16 && d.dtype != TX_BF16 && d.dtype != TX_F8E5M2)
    return fail(TX_ERR_UNSUPPORTED, "dtype %d: fp16, bf16 and fp8 e5m2 q/k/v/o are implemented",
                d.dtype);
  if (d.head_dim != 16 && d.head_dim != 32 && d.head_dim != 64 && d.head_dim != 128 &&
      d.head_dim != 256)
    return fail(TX_ERR_UNSUPPORTED, "head_dim %d: 16, 32, 64, 128 and 256 are implemented",
                d.head_dim);
  if (d.block_m == 0) d.block_m = 128;
  if (d.block_n == 0) d.block_n = 64;
  if ((d.block_m != 64 && d.block_m != 128) || (d.block_n != 32 && d.block_n != 64))
    return fail(TX_ERR_UNSUPPORTED, "blocks %dx%d: BLOCK_M 64 or 128 by BLOCK_N 32 or 64 "
                "are implemented", d.block_m, d.block_n);
  if (d.N_CTX % d.block_m)
    return fail(TX_ERR_UNSUPPORTED, "N_CTX %lld is not a multiple of %d (whole blocks only)",
                (long long)d.N_CTX, d.block_m);
  const bool fp8 = d.dtype == TX_F8E5M2;
  int rc = attnStrides(d, d.q_sz, d.q_sh, d.q_sm, "q", false);
  if (rc == TX_OK) rc = attnStrides(d, d.k_sz, d.k_sh, d.k_sm, "k", false);
  if (rc == TX_OK) rc = attnStrides(d, d.v_sz, d.v_sh, d.v_sm, "v", fp8);
  if (rc == TX_OK) rc = attnStrides(d, d.o_sz, d.o_sh, d.o_sm, "o", false);
  if (rc != TX_OK)
    return rc;
  const int64_t programs = d.Z * d.H * (d.N_CTX / d.block_m);
  if (programs > INT32_MAX || d.N_CTX > INT32_MAX / 2 || d.Z * d.H > INT32_MAX)
    return fail(TX_ERR_UNSUPPORTED, "grid above 2^31");
  std::memset(plan, 0, sizeof(*plan));
  plan->desc = d;
  const double zh = (double)d.Z * (double)d.H, n = (double)d.N_CTX;
  plan->flops = 4.0 * zh * n * n * d.head_dim * (d.causal ? 0.5 : 1.0);
  plan->bytes = 4.0 * zh * n * d.head_dim * (fp8 ? 1 : 2) + zh * n * 4;
  plan->qk_scale = d.sm_scale * 1.44269504f; // qk_scale = sm_scale; qk_scale *= 1.44269504
  plan->m_blocks = (int32_t)(d.N_CTX / d.block_m);
  plan->grid_x = (int32_t)programs;
  plan->block_threads = d.block_m / 32 * 64; // one wave per 32 query rows
  return TX_OK;
}

extern "C" TX_API int tx_attn_fwd_launch(const tx_attn_plan *plan, const void *q, const void *k,
                                         const void *v, void *o, float *M, void *stream) {
  g_last_error.clear();
  if (!plan)
    return fail(TX_ERR_INVALID, "plan is NULL");
  const tx_attn_desc &d = plan->desc;
  if (plan->grid_x == 0)
    return TX_OK;
  if (!q || !k || !v || !o || !M)
    return fail(TX_ERR_INVALID, "NULL tensor pointer");
  {
    // The plan comes back from the caller: planning its descriptor again
    // (host arithmetic) must give this plan, field for field, so that an
    // edited plan (strides, blocks, grid) never reaches the kernel.
    tx_attn_plan again;
    const int rc = tx_attn_fwd_plan(&d, &again);
    if (rc != TX_OK)
      return rc;
    // (field by field: the struct's tail padding carries no meaning)
    static_assert(sizeof(tx_attn_desc) == 3 * 8 + 4 * 4 + 12 * 8 + 2 * 4,
                  "tx_attn_desc has no padding");
    if (std::memcmp(&again.desc, &plan->desc, sizeof again.desc) != 0 ||
        again.flops != plan->flops || again.bytes != plan->bytes ||
        again.qk_scale != plan->qk_scale || again.m_blocks != plan->m_blocks ||
        again.grid_x != plan->grid_x || again.block_threads != plan->block_threads)
      return fail(TX_ERR_INVALID, "the plan does not follow from its descriptor");
  }
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
       reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(o)) & 15 ||
      reinterpret_cast<uintptr_t>(M) & 3)
    return fail(TX_ERR_INVALID, "q, k, v, o must be 16-byte aligned and M 4-byte aligned");
  const bool bm64 = d.block_m == 64, bn32 = d.block_n == 32;
  if ((d.block_m != 64 && d.block_m != 128) || (d.block_n != 32 && d.block_n != 64) ||
      plan->block_threads != d.block_m / 32 * 64 ||
      (d.head_dim != 16 && d.head_dim != 32 && d.head_dim != 64 && d.head_dim != 128 &&
       d.head_dim != 256) ||
      (d.dtype != TX_F16 && d.dtype != TX_BF16 && d.dtype != TX_F8E5M2) || d.N_CTX % d.block_m ||
      plan->m_blocks != d.N_CTX / d.block_m || plan->grid_x != d.Z * d.H * plan->m_blocks)
    return fail(TX_ERR_INVALID, "plan launch shape does not match the attention kernel");
  if (!tx_device_available())
    return fail(TX_ERR_NO_DEVICE, "no gfx950 device visible");
  txk::AttnArgs a;
  a.Q = q;
  a.K = k;
  a.V = v;
  a.O = o;
  a.M = M;
  a.q_sz = d.q_sz, a.q_sh = d.q_sh, a.q_sm = d.q_sm;
  a.k_sz = d.k_sz, a.k_sh = d.k_sh, a.k_sm = d.k_sm;
  a.v_sz = d.v_sz, a.v_sh = d.v_sh, a.v_sm = d.v_sm;
  a.o_sz = d.o_sz, a.o_sh = d.o_sh, a.o_sm = d.o_sm;
  a.H = (int32_t)d.H;
  a.N_CTX = (int32_t)d.N_CTX;
  a.qk_scale = plan->qk_scale;
  hipStream_t s = static_cast<hipStream_t>(stream);
  typedef void (*AttnFn)(txk::AttnArgs);
#define TX_ATTN_BLOCKS(C, HD, BF)                                                          \
  {{txk::attn_fwd_kernel<C, HD, BF, 128, 64>, txk::attn_fwd_kernel<C, HD, BF, 128, 32>},    \
   {txk::attn_fwd_kernel<C, HD, BF, 64, 64>, txk::attn_fwd_kernel<C, HD, BF, 64, 32>}}
#define TX_ATTN_DTYPES(C, HD) {TX_ATTN_BLOCKS(C, HD, false), TX_ATTN_BLOCKS(C, HD, true)}
  // [causal][head_dim 16 / 32 / 64 / 128 / 256][bf16][BLOCK_M 64][BLOCK_N 32]
  static const AttnFn kAttn[2][5][2][2][2] = {
      {TX_ATTN_DTYPES(false, 16), TX_ATTN_DTYPES(false, 32), TX_ATTN_DTYPES(false, 64),
       TX_ATTN_DTYPES(false, 128), TX_ATTN_DTYPES(false, 256)},
      {TX_ATTN_DTYPES(true, 16), TX_ATTN_DTYPES(true, 32), TX_ATTN_DTYPES(true, 64),
       TX_ATTN_DTYPES(true, 128), TX_ATTN_DTYPES(true, 256)}};
#undef TX_ATTN_DTYPES
#undef TX_ATTN_BLOCKS
  // [causal][head_dim 16 / 32 / 64 / 128 / 256][BLOCK_M 64][BLOCK_N 32]
#define TX_ATTN8_BLOCKS(C, HD)                                                             \
  {{txk::attn_fwd8_kernel<C, HD, 128, 64>, txk::attn_fwd8_kernel<C, HD, 128, 32>},          \
   {txk::attn_fwd8_kernel<C, HD, 64, 64>, txk::attn_fwd8_kernel<C, HD, 64, 32>}}
  static const AttnFn kAttn8[2][5][2][2] = {
      {TX_ATTN8_BLOCKS(false, 16), TX_ATTN8_BLOCKS(false, 32), TX_ATTN8_BLOCKS(false, 64),
       TX_ATTN8_BLOCKS(false, 128), TX_ATTN8_BLOCKS(false, 256)},
      {TX_ATTN8_BLOCKS(true, 16), TX_ATTN8_BLOCKS(true, 32), TX_ATTN8_BLOCKS(true, 64),
       TX_ATTN8_BLOCKS(true, 128), TX_ATTN8_BLOCKS(true, 256)}};
#undef TX_ATTN8_BLOCKS
  const int c = d.causal ? 1 : 0;
  const int hd = d.head_dim == 16    ? 0
                 : d.head_dim == 32  ? 1
                 : d.head_dim == 64  ? 2
                 : d.head_dim == 128 ? 3
                                     : 4;
  const AttnFn fn = d.dtype == TX_F8E5M2 ? kAttn8[c][hd][bm64][bn32]
                                         : kAttn[c][hd][d.dtype == TX_BF16][bm64][bn32];
  hipLaunchKernelGGL(fn, dim3(plan->grid_x), dim3(plan->block_threads), 0, s, a);
  TX_HIP_CHECK(hipGetLastError());
  return TX_OK;
}

#define TRITON_EXT_ARG "tx-mi355x-dot"
#define TRITON_EXT_RUN txMi355xDotRun
#include "../../infra/TritonExtPass.inc"
