// arith_intensity extension: libarith_intensity.so.
//
// The task names an "arithmetic-intensity pass" that the reference snapshot
// does not contain, so this extension has no reference source to follow.  It
// classifies a dot by its algorithmic work (every operand read once, the
// output written once, scales read once) against MI355X's roofline and
// recommends a tile from the set the mi355x_dot backend instantiates.
//
// MI355X public dense peaks: bf16/fp16 MFMA 2516.6 TFLOP/s (256 CUs x
// 2.4 GHz x 4096 FLOP/clk/CU), fp8 and int8 5033.2 T(FL)OP/s, fp4 10066.4
// TFLOP/s, HBM3E 8 TB/s.

#include "triton_ext/TritonExtPassInfra.h"
#include "triton_ext/tx_dot.h"
#include "triton_ext/tx_passes.h"

#include <climits>
#include <cmath>
#include <cstdint>

namespace {

constexpr double kPeak16 = 2516.6e12;
constexpr double kPeak8 = 5033.2e12;
constexpr double kPeak4 = 10066.4e12;
constexpr double kPeakF32 = 157.3e12;
constexpr double kHbm = 8.0e12;
constexpr int kCUs = 256;

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

struct Tile {
  int32_t bm, bn, bk;
  double eff;  // fraction of MFMA peak a tile of this size sustains
  int occ = 1; // workgroups per CU that eff needs (latency hidden by each other)
};

// Tiles the backend instantiates, largest first.  `eff` is the fraction of
// the dense MFMA peak each tile sustained at 4096^3 on one MI355X (bench.py
// --only tiles: bf16 -> bf16 and int8 -> int32, back-to-back launches):
// 16-bit 256x256x64 0.509, 128x128x64 0.341, 64x64x32 0.187; 8-bit
// 256x256x128 0.463, 128x128x128 0.173.  tileCost weighs them against the
// waves of tiles a shape needs.
// With fewer workgroups than occ per CU a tile runs at the rate of occ per
// CU all the same (measured at M = 128 / 512, N = K = 8192: 64x64x32 190 us,
// 128x128x64 154 us, where eff alone predicts 36 and 80).
const Tile kTiles16[] = {{256, 256, 64, 0.509, 1}, {128, 128, 64, 0.341, 2},
                         {64, 64, 32, 0.187, 4}};
// 8-bit tiles.  (A 256x224 tile also exists for explicit requests: it fills
// all CUs at N = 7168, but its A-resident wave layout needs 28 transposed B
// reads per step against 16; it measured 0.273 at int8 4096^3 and no faster
// than 256x256 at N = 7168.)
const Tile kTiles8[] = {{256, 256, 128, 0.463, 1}, {128, 128, 128, 0.173, 2}};
// MX (tl.dot_scaled) tiles: one 256x256 tile of 128 bytes of K per step,
// i.e. 128 fp8 or 256 fp4 elements.
const Tile kTileMx8 = {256, 256, 128, 0.45}, kTileMx4 = {256, 256, 256, 0.33};

// Estimated time of a tiled dot in MAC-units of one CU: whole waves of
// occ workgroups a CU, each a tile over its K range costing BM*BN*K / eff.  The 256x256 tiles split K when they leave most CUs idle
// (tx_gemm_split_k): the ranges run as more workgroups, and their fp32
// partials, written and read back (8 S M N bytes), add their HBM time and a
// second launch at `cu_macs` (a CU's peak MAC rate).
double tileCost(const Tile &t, int64_t M, int64_t N, int64_t K, double cu_macs) {
  const int64_t tiles = cdiv(M, t.bm) * cdiv(N, t.bn);
  const int64_t ksteps = cdiv(K, t.bk);
  const int32_t s = t.bm == 256 && t.bn == 256 ? tx_gemm_split_k(tiles, ksteps) : 1;
  const int64_t waves = cdiv(tiles * s, (int64_t)kCUs * t.occ) * t.occ;
  double c = (double)waves * t.bm * t.bn * (double)cdiv(ksteps, s) * t.bk / t.eff;
  if (s > 1)
    c += (8.0 * s * (double)M * (double)N / kHbm + 4e-6) * cu_macs;
  return c;
}

// Cheapest candidate from index `first` on (the 256-wide tile is index 0).
template <size_t N>
Tile chooseTile(const Tile (&cands)[N], int64_t M, int64_t Nn, int64_t K, double cu_macs,
                size_t first = 0) {
  Tile best = cands[first];
  double bestCost = tileCost(best, M, Nn, K, cu_macs);
  for (size_t i = first + 1; i < N; ++i) {
    double c = tileCost(cands[i], M, Nn, K, cu_macs);
    if (c < bestCost) {
      best = cands[i];
      bestCost = c;
    }
  }
  return best;
}

} // namespace

extern "C" int32_t tx_gemm_split_k(int64_t tiles, int64_t ksteps) {
  int32_t s = 1;
  while (s < 16 && tiles * s * 2 <= kCUs && ksteps / (s * 2) >= 8)
    s *= 2;
  return s;
}

extern "C" int32_t tx_dtype_bits(int32_t dtype) {
  switch (dtype) {
  case TX_F32: return 32;
  case TX_F16: return 16;
  case TX_BF16: return 16;
  case TX_I8: return 8;
  case TX_F8E4M3: return 8;
  case TX_I32: return 32;
  case TX_F8E5M2: return 8;
  case TX_F4E2M1: return 4;
  default: return 0;
  }
}

extern "C" int32_t tx_dtype_size(int32_t dtype) {
  const int32_t b = tx_dtype_bits(dtype);
  return b % 8 ? 0 : b / 8;
}

extern "C" double tx_mi355x_peak_flops(int32_t dtype) {
  switch (dtype) {
  case TX_F16:
  case TX_BF16: return kPeak16;
  case TX_I8:
  case TX_F8E4M3:
  case TX_F8E5M2: return kPeak8;
  case TX_F4E2M1: return kPeak4;
  case TX_F32: return kPeakF32;
  default: return 0.0;
  }
}

extern "C" double tx_mi355x_peak_bw(void) { return kHbm; }

extern "C" int tx_dot_operand_spans(const tx_dot_desc *d, int64_t *a_bytes, int64_t *b_bytes) {
  if (!d || !a_bytes || !b_bytes)
    return TX_ERR_INVALID;
  const int32_t ba = tx_dtype_bits(d->a_type), bb = tx_dtype_bits(d->b_type);
  if (!ba || !bb)
    return TX_ERR_INVALID;
  const bool bt = (d->flags & TX_FLAG_B_KMAJOR) != 0;
  const int64_t lda = d->lda ? d->lda : d->K;
  const int64_t ldb = d->ldb ? d->ldb : (bt ? d->K : d->N);
  // ((rows - 1) * ld + len) elements of `bits` bits, in 128-bit arithmetic
  auto span = [](int64_t rows, int64_t ld, int64_t len, int32_t bits) -> int64_t {
    if (rows <= 0 || len <= 0)
      return 0;
    const __int128 e = (__int128)(rows - 1) * ld + len;
    const __int128 b = (e * bits + 7) / 8;
    return b > (__int128)INT64_MAX ? INT64_MAX : (int64_t)b;
  };
  *a_bytes = span(d->M, lda, d->K, ba);
  if (bt)
    *b_bytes = span(d->N, ldb, d->K, bb);
  else if (bb == 4) // packed rows of two K values: K / 2 rows of ldb bytes
    *b_bytes = span((d->K + 1) / 2, ldb, d->N, 8);
  else
    *b_bytes = span(d->K, ldb, d->N, bb);
  return TX_OK;
}

extern "C" int tx_arith_intensity(const tx_dot_desc *d, tx_ai_report *out) {
  if (!d || !out)
    return TX_ERR_INVALID;
  *out = tx_ai_report{};
  const int32_t ba = tx_dtype_bits(d->a_type), bb = tx_dtype_bits(d->b_type),
                bc = tx_dtype_bits(d->c_type);
  if (!ba || !bb || !bc || d->M < 0 || d->N < 0 || d->K < 0)
    return TX_ERR_INVALID;
  const double sa = ba / 8.0, sb = bb / 8.0, sc = bc / 8.0; // bytes per element
  const double M = (double)d->M, N = (double)d->N, K = (double)d->K;
  double scaleBytes = 0.0;
  if (d->scale_mode == TX_SCALE_ROWCOL)
    scaleBytes = 4.0 * (M + N);
  else if (d->scale_mode == TX_SCALE_BLOCK128)
    scaleBytes = 4.0 * (M * cdiv(d->K, 128) +
                        (double)cdiv(d->K, 128) * cdiv(d->N, 128));
  else if (d->scale_mode == TX_SCALE_MX32 || d->scale_mode == TX_SCALE_NV16)
    // one scale byte per 32 K (e8m0) or 16 K (e4m3); a bf16 side has none
    scaleBytes = ((ba == 16 ? 0.0 : M) + (bb == 16 ? 0.0 : N)) *
                 (double)cdiv(d->K, d->scale_mode == TX_SCALE_NV16 ? 16 : 32);
  out->flops = 2.0 * M * N * K;
  // C once, twice when accumulating into it (read, then written)
  const double cPasses = (d->flags & TX_FLAG_ACCUMULATE) ? 2.0 : 1.0;
  out->bytes = M * K * sa + K * N * sb + cPasses * M * N * sc + scaleBytes;
  out->intensity = out->bytes > 0 ? out->flops / out->bytes : 0.0;
  // a mixed product runs at the rate of its wider operand
  out->peak_flops = ba >= bb ? tx_mi355x_peak_flops(d->a_type)
                             : tx_mi355x_peak_flops(d->b_type);
  if (d->scale_mode == TX_SCALE_NV16) // e4m3 scales run on the bf16 tile
    out->peak_flops = tx_mi355x_peak_flops(TX_BF16);
  out->peak_bw = kHbm;
  out->ridge = out->peak_flops / out->peak_bw;
  out->bound = out->intensity > out->ridge ? TX_BOUND_MFMA : TX_BOUND_HBM;
  double tc = out->peak_flops > 0 ? out->flops / out->peak_flops : 0.0;
  double tm = out->bytes / out->peak_bw;
  out->roofline_us = 1e6 * (tc > tm ? tc : tm);

  Tile t{d->block_m, d->block_n, d->block_k, 1.0};
  if (t.bm <= 0 || t.bn <= 0 || t.bk <= 0) {
    // Operands as the tile reads them (an upcast MX side: packed bf16), and
    // whether the 256-wide tiles (32-bit buffer offsets) can address them.
    const bool upcast = (d->scale_mode == TX_SCALE_MX32 && (ba == 16 || bb == 16)) ||
                        d->scale_mode == TX_SCALE_NV16;
    tx_dot_desc e = *d;
    if (upcast) {
      if (e.a_type != TX_BF16)
        e.a_type = TX_BF16, e.lda = 0;
      if (e.b_type != TX_BF16)
        e.b_type = TX_BF16, e.ldb = TX_MX_UPCAST_LD(d->N);
    }
    int64_t spanA = 0, spanB = 0;
    tx_dot_operand_spans(&e, &spanA, &spanB);
    // The decode kernels' epilogues: W8A8 (row x column scales, bf16 C) and
    // the plain int8 -> int32 dot (no scales, int32 C), N up to their 4096
    // column strips; B row-major, or K-major on the row kernel (M > 48: the
    // 8-bit ring decode kernel takes K-major B below that).  Both stream B
    // once with split-K.
    const bool decode =
        d->a_type == TX_I8 && d->b_type == TX_I8 &&
        (!(d->flags & TX_FLAG_B_KMAJOR) || d->M > 48) && d->N <= (int64_t)4096 * 128 &&
        ((d->scale_mode == TX_SCALE_ROWCOL && d->c_type == TX_BF16) ||
         (d->scale_mode == TX_SCALE_NONE && d->c_type == TX_I32));
    // The 16-bit decode kernel: both operands bf16 or both fp16, no scales,
    // C in their type or fp32, B row-major or K-major, M <= 96, N up to its
    // 16384 strips of 64 columns.  It streams B once with split-K.  Each wave
    // reads every row of the slice from LDS, so its time grows with M: at
    // N = K = 8192 bf16, M = 80 / 96 / 112 / 128 44.1 / 48.6 / 53.9 / 57.6 us
    // against the 256 tile with split-K's 51.9 / 51.9 / 54.1 / 56.6.
    const bool decode16 =
        (d->a_type == TX_BF16 || d->a_type == TX_F16) && d->b_type == d->a_type &&
        d->scale_mode == TX_SCALE_NONE && (d->c_type == d->a_type || d->c_type == TX_F32) &&
        d->M <= 96 && d->N <= (int64_t)16384 * 64;
    // The 8-bit ring decode kernel, B row-major or K-major: fp8 x fp8 with
    // fp32 C, e4m3 x e4m3 with 128-block scales and bf16 / fp32 C, M <= 64;
    // with B K-major also int8 -> int32 and W8A8, M <= 48 (the row kernel's
    // 32 x 32 x 32 products take M = 64: W8A8 22.4 against 26.8 us at
    // N = K = 8192); N up to its 16384 strips of 128 columns.
    const bool fp8a = d->a_type == TX_F8E4M3 || d->a_type == TX_F8E5M2;
    const bool fp8b = d->b_type == TX_F8E4M3 || d->b_type == TX_F8E5M2;
    const bool kmajor = (d->flags & TX_FLAG_B_KMAJOR) != 0;
    const bool decode_f8 =
        d->M <= 64 && d->N <= (int64_t)16384 * 128 &&
        ((fp8a && fp8b && d->scale_mode == TX_SCALE_NONE && d->c_type == TX_F32) ||
         (d->scale_mode == TX_SCALE_BLOCK128 && d->a_type == TX_F8E4M3 &&
          d->b_type == TX_F8E4M3 && (d->c_type == TX_BF16 || d->c_type == TX_F32)) ||
         (kmajor && d->a_type == TX_I8 && d->b_type == TX_I8 && d->M <= 48 &&
          ((d->scale_mode == TX_SCALE_NONE && d->c_type == TX_I32) ||
           (d->scale_mode == TX_SCALE_ROWCOL && d->c_type == TX_BF16))));
    const size_t first = spanA < TX_SPAN32_LIMIT && spanB < TX_SPAN32_LIMIT ? 0 : 1;
    if (upcast)
      t = chooseTile(kTiles16, d->M, d->N, d->K, kPeak16 / 2 / kCUs, first); // MX x bf16: bf16 tile
    else if (d->scale_mode == TX_SCALE_MX32)
      t = ba == 4 ? kTileMx4 : kTileMx8;
    else if (decode_f8)
      t = Tile{(int32_t)(16 * cdiv(d->M > 0 ? d->M : 1, 16)), 128, 128, 1.0};
    else if (decode16) {
      // Every strip reads all of A, so A's re-reads are M / W of B's bytes.
      // Strips of W = 128 columns halve them: at N = K = 8192 bf16 M = 48 / 64
      // / 80 31.3 / 34.0 / 38.0 us against 35.0 / 39.6 / 45.3 with 64 (B
      // K-major: M = 32 28.5 against 31.8), about equal at M = 16; M = 64 at
      // N = 16384 / 28672 57.1 / 100.2 against 68.4 / 129.9.  With B under
      // 2^25 elements the wider strips double the split (and its partials) or
      // halve the workgroups, and lose: M = 64 at N = K = 4096 18.2 against
      // 16.4 us, at N = 2048 22.0 against 17.9.  Their ring holds slices up
      // to 80 rows.  Slices of 16 rows gain from them at N >= 16384, where 64
      // columns make 256 strips or more: M = 16 at N = 28672, K = 8192 77.6
      // against 93.0 us (B K-major 73.6 / 87.4), at N = 16384, K = 4096 26.6
      // against 28.9 (K-major 29.3 / 37.0); at N = K = 8192 they tie.
      const int32_t rows = (int32_t)(16 * cdiv(d->M > 0 ? d->M : 1, 16));
      const int64_t nk = d->N * d->K;
      const bool wide = (rows >= 32 && rows <= 80 && nk >= ((int64_t)1 << 25)) ||
                        (rows == 16 && d->N >= 16384 && nk >= ((int64_t)1 << 26));
      t = Tile{rows, wide ? 128 : 64, 128, 1.0};
    }
    else if (sa == 2 && (d->flags & TX_FLAG_B_KMAJOR))
      t = kTiles16[0]; // the K-major B kernel exists for this tile only
    else if (sa == 2)
      t = chooseTile(kTiles16, d->M, d->N, d->K, kPeak16 / 2 / kCUs, first);
    else if (decode && d->M <= 256)
      // W8A8 decode (M <= 256, N up to its 4096 column strips; past it the
      // 8-bit tiles with split-K: at N = K = 8192 M = 384 57.5 us, 512 63.9,
      // against 76.0 and 78.7 for the row kernel's slices of 256), 128-column
      // strips.  Up to M = 48 one row slice and 64-row K batches split among
      // the waves; beyond, row slices whose waves all take every 128-row K
      // batch: of 64 rows up to M = 128, of 128 past it.  Measured at
      // N = K = 8192, in us: M = 32 20.1 / 22.1-22.7 (slices of 64), 48 22.0 /
      // 22.2-22.5, 64 25.2 / 22.3-22.9, 96 29.4 (64) / 31.2-32.0 (128), 128
      // 29.6 / 30.5, 192 53.5 / 43.7-44.8, 256 44.8 / 42.6.
      t = d->M > 128 ? Tile{128, 128, 128, 1.0}
          : d->M > 48 ? Tile{64, 128, 128, 1.0}
                      : Tile{(int32_t)(16 * cdiv(d->M > 0 ? d->M : 1, 16)), 128, 64, 1.0};
    else if (d->flags & TX_FLAG_B_KMAJOR)
      t = kTiles8[0]; // of the 8-bit tiles only this one has a K-major B form
    else if (d->a_type == TX_F8E4M3 || d->a_type == TX_F8E5M2)
      t = kTiles8[first]; // the register-staged 128x128 tile is slower everywhere
    else
      t = chooseTile(kTiles8, d->M, d->N, d->K, kPeak8 / 2 / kCUs, first);
  }
  out->block_m = t.bm;
  out->block_n = t.bn;
  out->block_k = t.bk;
  out->tile_intensity = 2.0 * t.bm * t.bn / ((double)(t.bm + t.bn) * sa);
  return TX_OK;
}

namespace {

// Pass body: classification and tile choice for one dot.
int txArithIntensityRun(tx_dot_plan *plan) {
  tx_ai_report r;
  int rc = tx_arith_intensity(&plan->desc, &r);
  if (rc != TX_OK)
    return rc;
  plan->flops = r.flops;
  plan->bytes = r.bytes;
  plan->intensity = r.intensity;
  plan->peak_flops = r.peak_flops;
  plan->peak_bw = r.peak_bw;
  plan->ridge = r.ridge;
  plan->roofline_us = r.roofline_us;
  plan->tile_intensity = r.tile_intensity;
  plan->bound = r.bound;
  plan->desc.block_m = r.block_m;
  plan->desc.block_n = r.block_n;
  plan->desc.block_k = r.block_k;
  plan->passes_run += 1;
  return TX_OK;
}

} // namespace

#define TRITON_EXT_ARG "tx-arith-intensity"
#define TRITON_EXT_RUN txArithIntensityRun
#include "../../infra/TritonExtPass.inc"
