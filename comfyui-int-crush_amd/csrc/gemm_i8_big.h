// INT8-MFMA GEMM on 256/288/320 x 192 output tiles (gfx950), for shapes whose
// 256 x 128 / 256 x 256 tilings end in a partly filled round of workgroups.
// The weight modes share the tile, the DMA ring and the epilogue (the W4A16
// modes, at the enum below, put fp16 MFMAs on the same layout):
//  * grouped INT4, the arithmetic of gemm_i8_kernel's grouped path
//    (triton_w4a8_gemm.py:40-108 with the per-group scales of
//    _quant_utils.py:237-270): per 128-column stage (or 64- or 32-column
//    step) an exact int32 block sum of 16*q weights, folded in group order as
//    facc = fma(f32(acc_g), s_w[n, g] / 16, facc); out = facc * s_a[m] (+ bias);
//  * per-row INT4 and per-row INT8 (triton_int8_gemm.py:46-205): int32 sums
//    over all of K, out = f32(acc) [/ 16] * (s_a[m] * s_w[n]) (+ bias).
// Every mode rounds once and is bit-identical to gemm_i8_kernel.
//
// The row count is a template parameter: 256, 288 or 320 (8, 9 or 10 blocks of
// 16 rows per wave), whichever tiles M in the fewest rounds.
//
// Why this tile: a round of workgroups costs the same whether all CUs are busy
// or a few, and 4608 x 3072 (the Flux MLP-down / C3 shape) makes 432 tiles of
// 256 x 128 on 256 CUs, 1.69 rounds paid as two.  4608 x 3072 / 256 CUs is
// 2^11 * 27 outputs per CU, and 288 x 192 is the one tile of that area whose
// sides divide M and N with 16-row / 16-column blocks: 16 x 16 tiles, one
// round.  Its operands per 128-K stage (36 KB of activations, 12 KB of packed
// weights) are 0.87 bytes per output against 1.22 for 256 x 128.
//
// The price is registers: 288 x 192 outputs over 512 lanes are 108 per lane.
// Holding an int32 group sum and an fp32 running sum for each (216 VGPRs)
// leaves too little for the operands, so here only the fp32 sums are
// resident: each 16 x 16 block runs both 64-K steps of a stage back to back
// and is folded right after, its group sum held only meanwhile.
//
// Layout: 8 waves in 2 (rows) x 4 (columns), each owning 144 x 48 = 9 x 3
// blocks of v_mfma_i32_16x16x64_i8.  Operand lane l holds 16 K-bytes (chunk
// l/16 of the 64-K step) of row / column l%16, the same chunk for both
// operands, so the K order inside the instruction does not matter; result
// lane l holds rows 4*(l/16) + r (r = 0..3) of column l%16.  Activations,
// packed weights and scales reach LDS by DMA through a two-slot ring (the
// activation rows swizzled as in gemm_i8_kernel).  Each wave expands its own
// weight fragments from the packed slot into registers (8 packed bytes per
// lane and fragment), so no expanded tile is written to LDS and a stage needs
// one barrier, not two; the two waves of a column group expand the same
// fragments (60 VALU instructions per wave and stage against 30 for a shared
// expansion, which measured 4 % slower with its extra barrier and LDS
// round trip).  Measured at C3 (4608 x 3072 x 12288): 256 x 128 tiles 273 us,
// this tile with a shared expansion 227 us, with register expansion 217 us,
// plus the priority ramp below 208 us.
//
// Wave priorities: the two waves on a SIMD (one per wave row) run the same
// instruction mix, MFMAs and the fold's VALU work, and the arbiter favours the
// older one, which finished its rows of a stage in ~2700 shader clocks while
// the younger took ~3900 and the older idled at the barrier.  Each wave
// therefore steps its priority down over the block rows (3 3 2 2 1 1 0 0 0):
// a wave that runs ahead yields the SIMD to the one behind.
#pragma once
#include <type_traits>

#include "dequant4.h"
#include "gemm_common.h"

namespace {
namespace big {
// Weight modes: grouped INT4 folded per 128-column stage, grouped INT4 folded
// per 64-column step, per-row INT4, per-row INT8 (no fold: int32 sums across
// K), grouped INT4 folded per 32-column half step, grouped int8 folded per
// 128-column stage (INT4 weights unpacked once to one byte each: no
// expansion in the main loop, twice the weight bytes per stage), and W4A16:
// 16-bit activations, INT4 weights dequantized in registers to RN_dt(q *
// RN_dt(s)) and summed in fp32 by v_mfma_f32_16x16x32_{f16,bf16} (64-K
// stages: the same 128-byte LDS rows and 16-byte fragments as the int8
// modes), with a two-slot ring (W16) or a three-slot one (W16L, long K), on
// 192-column tiles or (W16X, W16LX) 256-column ones: four 16-column blocks
// per wave, a quarter fewer activation bytes per output
enum { G128 = 0, G64 = 1, ROW4 = 2, ROW8 = 3, G32 = 4, G128I8 = 5, W16 = 6, W16L = 7, W16X = 8, W16LX = 9 };
constexpr int BN = 192, NS = 2;
constexpr int TNB = 3;                       // 16 x 16 blocks per wave in N
constexpr int WCOLS = TNB * 16;
constexpr int S_BYTES = BN * 4;              // one fp32 scale per column and scale block
constexpr int S_WAVES = BN / 64;             // waves issuing a scale DMA
constexpr int EPI_RS = BN + 8;               // 16-bit output staging row stride
// Tile rows: TMB 16-row blocks per wave, two wave rows (256, 288 or 320 rows
// for TMB = 8, 9, 10)
template <int TMB_, int MODE_>
struct Rows {
  static constexpr int TMB = TMB_, MODE = MODE_;
  static constexpr bool GROUPED = MODE <= G64 || MODE == G32 || MODE == G128I8, F64 = MODE == G64, F32 = MODE == G32;
  static constexpr bool INT8W = MODE == ROW8 || MODE == G128I8;
  static constexpr bool DEQ = MODE >= W16;  // W4A16: one scale row per 64-K stage, no fold
  static constexpr bool WIDE = MODE == W16X || MODE == W16LX;
  // tile columns and the quantities that follow from them (hiding big::BN ...)
  static constexpr int BN = WIDE ? 256 : big::BN;
  static constexpr int TNB = BN / 64, WCOLS = TNB * 16, S_BYTES = BN * 4, S_WAVES = BN / 64, EPI_RS = BN + 8;
  static constexpr bool SCALED = GROUPED || DEQ;  // the slot holds scale rows
  static constexpr int KS = DEQ ? 64 : kBK;       // K values per stage
  // ring slots: W16L keeps two DMA stages in flight in a three-slot ring
  // (W4A16's stages are short: one barrier, no fold), the other modes one in
  // two.  Measured on MI355X: 4608 x 3072 x 12288 (one round, 192 stages)
  // 359 -> 322 us; C2 4608 x 12288 x 3072 (four rounds of 48 stages, each
  // tile paying the deeper prologue) 310 -> 319 us.
  static constexpr int NSL = MODE == W16L || MODE == W16LX ? 3 : NS;
  static constexpr int NSC = F32 ? 4 : (F64 ? 2 : 1);  // scale rows per stage (grouped)
  static constexpr int BM = 32 * TMB, WROWS = 16 * TMB;
  static constexpr int A_BYTES = BM * kBK;
  static constexpr int A_BLOCKS = BM / 8;             // 1 KB DMA blocks: 8 rows of 128 bytes
  static constexpr int A_PER = (A_BLOCKS + 7) / 8;    // blocks per wave
  // weights per stage: packed nibbles (1 KB DMA blocks of 16 rows of 64
  // bytes) or int8 (blocks of 8 rows of 128 bytes, swizzled as the activations)
  static constexpr int B_BYTES = INT8W ? BN * kBK : BN * KS / 2;
  static constexpr int B_BLOCKS = B_BYTES / 1024;
  static constexpr int B_PER = (B_BLOCKS + 7) / 8;
  // ring slot: activations, weights, then none, one (scale blocks of 128
  // columns), two (of 64) or four (of 32) scale rows
  static constexpr int SLOT = A_BYTES + B_BYTES + (SCALED ? NSC * S_BYTES : 0);
  // staging tile, activation scales, bias and per-row weight scales
  static constexpr size_t epi_bytes = (size_t)BM * EPI_RS * 2 + (size_t)(BM + 2 * BN) * 4;
  static constexpr size_t lds_bytes = (size_t)NSL * SLOT > epi_bytes ? (size_t)NSL * SLOT : epi_bytes;
  // wave priority per block row: 3 3 2 2 1 1 0 0 ...
  static constexpr int prio(int i) { return i < 6 ? 3 - i / 2 : 0; }
  static_assert(SLOT % 16 == 0 && lds_bytes <= 160 * 1024, "LDS layout");
  static_assert(4 * WCOLS == BN, "wave grid");
  static_assert(A_PER + B_PER <= TMB, "one DMA slot per block row");
};

typedef _Float16 v8h16 __attribute__((ext_vector_type(8)));
typedef __bf16 v8bf16 __attribute__((ext_vector_type(8)));
// fp32 += 16-bit A (rows) x 16-bit B (columns) over 32 K, operands as 16 bytes per lane
template <int DT> IC_DEV v4f mfma16(const v4i& a, const v4i& b, const v4f& c) {
  if constexpr (DT == IC_DTYPE_F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h16, a), __builtin_bit_cast(v8h16, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf16, a), __builtin_bit_cast(v8bf16, b), c, 0,
                                                   0, 0);
}
}  // namespace big

// F64: groups of 64 columns, or of an odd multiple of 64 (gcd(group, 128)
// = 64): each 64-K step is folded by itself, with the scale of its group, so
// a stage folds twice.  F32: groups of an odd multiple of 32 columns: each
// 64-K step runs as two MFMAs on the activation fragments with the lanes of
// the other 32-column half zeroed (lanes 0-31 hold K 0-31 of the step, lanes
// 32-63 K 32-63), so a stage folds four sums.  Otherwise (group sizes that
// are multiples of 128) each 128-column stage is folded once with its
// group's scale.
//
// ROW4 / ROW8: one scale per output column; the int32 sums run across all of K
// in the MFMAs (16 * q for INT4) and the epilogue forms
// f32(acc) [/ 16] * (s_a[m] * s_w[n]), as gemm_i8_kernel's per-row path.
//
// KIL: packed INT4 rows in the K-interleaved nibble order, whose expansion
// needs no byte permutes (3 instead of 5 VALU instructions per 8 weights).
// In the W4A16 modes KIL selects the staged operand layout instead: packed
// weights stage-major ([K/64][N][32 bytes], ldb = bytes between stages) and
// scales group-major ([G][N]), so that a stage's weight block of a tile is
// one contiguous 6 KB run and its 192 scales are 768 contiguous bytes.  In
// the row-major layouts the weight DMA touches 32 cache lines per KB (32 of
// each line's 128 bytes) and the scale DMA 64 lines per 256 bytes; the DMA
// path is paced by lines, not bytes (measured at C2 4608 x 12288 x 3072
// f16: 306 us, 275 us without the scale DMAs, 255 us without both).
template <int OUT_DT, bool EPI, int MODE, int TMB, bool KIL = false>
__global__ __launch_bounds__(kNT, 1) void gemm_i8_big_kernel(
    const int8_t* __restrict__ A, int64_t lda, const uint8_t* __restrict__ B, int64_t ldb,
    const float* __restrict__ s_a, const float* __restrict__ s_w, int G,
    const void* __restrict__ bias, int bias_dt, void* __restrict__ C, int64_t ldc, int M, int N,
    int K, ic_epi epi) {
  using namespace big;
  using RT = Rows<TMB, MODE>;
  // tile width and its derived quantities of this mode (hide big::BN ...)
  constexpr int BN = RT::BN, TNB = RT::TNB, WCOLS = RT::WCOLS, S_BYTES = RT::S_BYTES, S_WAVES = RT::S_WAVES,
                EPI_RS = RT::EPI_RS;
  constexpr int BM = RT::BM, WROWS = RT::WROWS, A_BYTES = RT::A_BYTES, A_BLOCKS = RT::A_BLOCKS;
  constexpr int A_PER = RT::A_PER, B_BYTES = RT::B_BYTES, B_BLOCKS = RT::B_BLOCKS, B_PER = RT::B_PER;
  constexpr bool GROUPED = RT::GROUPED, F64 = RT::F64, F32 = RT::F32, INT8W = RT::INT8W;
  constexpr bool DEQ = RT::DEQ, SCALED = RT::SCALED;
  constexpr int KS = RT::KS;
  constexpr int NS = RT::NSL;  // ring slots of this mode (hides big::NS)
  constexpr int LA = NS - 1;   // stages of DMAs in flight ahead of the one computed
  static_assert(OUT_DT != IC_DTYPE_F32, "16-bit outputs only");
  static_assert(!(KIL && INT8W), "the nibble order applies to packed INT4 weights");
  constexpr bool STAGED = DEQ && KIL;  // W4A16: stage-major weights, group-major scales
  constexpr int SLOT = RT::SLOT;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_char*)smem;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = wave >> 2, wc = wave & 3;
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int tm, tn;
  tile_coords(blockIdx.x, tiles_m * tiles_n, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  // epilogue operands (activation scale of row m0 + tid, bias of column
  // n0 + tid), loaded now so that their latency passes under the main loop
  static_assert(BM <= kNT && BN <= kNT, "one epilogue operand per thread");
  const float pre_sa = !DEQ && tid < BM ? s_a[min(m0 + tid, M - 1)] : 0.0f;
  const float pre_b = tid < BN && bias != nullptr ? ld_any_f32(bias, bias_dt, min(n0 + tid, N - 1)) : 0.0f;
  const float pre_sw = !GROUPED && !DEQ && tid < BN ? s_w[min(n0 + tid, N - 1)] : 0.0f;
  const int KT = K / KS;
  // scale blocks (of 128, 64 or 32 columns) per group
  const int bpg = (K / G) / (F32 ? 32 : (F64 || DEQ ? 64 : kBK));

  // ---- DMA addressing (rows past M or N re-read the last row; never stored).
  // A (and int8 B) block b: LDS rows 8b + l/8, chunk slot l%8 holding global
  // chunk (l%8) ^ swz(row).  Packed B block b: rows 16b + l/4, 16-byte parts.
  uint32_t a_off[A_PER], b_off[B_PER];
#pragma unroll
  for (int c = 0; c < A_PER; ++c) {
    const int row = 8 * (wave + 8 * c) + (lane >> 3);
    a_off[c] = (uint32_t)(min(row, M - 1 - m0) * lda + (((lane & 7) ^ swz(row)) << 4));
  }
#pragma unroll
  for (int c = 0; c < B_PER; ++c) {
    if constexpr (INT8W) {
      const int row = 8 * (wave + 8 * c) + (lane >> 3);
      b_off[c] = (uint32_t)(min(row, N - 1 - n0) * ldb + (((lane & 7) ^ swz(row)) << 4));
      continue;
    }
    if constexpr (DEQ) {
      // 32 packed bytes per row and 64-K stage: LDS part p of row n holds
      // global part p ^ bit 3 of n, so the fragment reads (4 bytes at 4c of
      // one part, 16 rows) cover all 64 banks
      const int row = 32 * (wave + 8 * c) + (lane >> 1);
      b_off[c] = (uint32_t)(min(row, N - 1 - n0) * (STAGED ? 32 : ldb) + (((lane & 1) ^ ((row >> 3) & 1)) << 4));
      continue;
    }
    // packed row n (64 bytes) holds its 16-byte part p at part p ^ ((n >> 2) & 3):
    // the fragment reads of 16 consecutive rows then spread over all banks
    const int row = 16 * (wave + 8 * c) + (lane >> 2);
    const int part = (lane & 3) ^ ((lane >> 4) & 3);
    b_off[c] = (uint32_t)(min(row, N - 1 - n0) * ldb + (part << 4));
  }
  // scale DMA: a dword per lane and column, or (staged layout) one dwordx4
  // DMA of 48 lanes over the tile's 192 contiguous scales, from wave 7, which
  // issues the fewest activation and weight DMAs (N is a multiple of 8 there,
  // so the clamped 4-column chunks stay in the row)
  const uint32_t s_off = STAGED ? (uint32_t)(min(4 * lane, N - 4 - n0) * 4)
                                : (uint32_t)(min(64 * wave + lane, N - 1 - n0) * G * 4);
  const bool s_wave = STAGED ? wave == 7 : wave < S_WAVES;
  const int8_t* a_base = A + (int64_t)m0 * lda;
  const uint8_t* b_base = B + (int64_t)n0 * (STAGED ? 32 : ldb);
  const float* s_base = s_w + (int64_t)n0 * (STAGED ? 1 : G);

  auto slot_of = [&](int kt) { return lds0 + (uint32_t)((kt % NS) * SLOT); };
  auto dma_a = [&](int kt, int c) {
    const int blk = wave + 8 * c;  // wave-uniform
    if (blk < A_BLOCKS) dma16(a_off[c], a_base + (int64_t)kt * kBK, slot_of(kt) + (uint32_t)(blk * 1024));
  };
  auto dma_b = [&](int kt, int c) {
    const int blk = wave + 8 * c;
    if (blk < B_BLOCKS)
      dma16(b_off[c], b_base + (int64_t)kt * (INT8W ? kBK : (STAGED ? ldb : KS / 2)),
            slot_of(kt) + (uint32_t)(A_BYTES + blk * 1024));
  };
  auto dma_s = [&](int kt) {
    if (SCALED && s_wave) {
      if constexpr (STAGED) {
        if (lane < BN / 4)
          dma16(s_off, s_base + (int64_t)(kt / bpg) * N, slot_of(kt) + (uint32_t)(A_BYTES + B_BYTES));
      } else if constexpr (F32) {
#pragma unroll
        for (int h = 0; h < 4; ++h)
          dma4(s_off, s_base + (4 * kt + h) / bpg,
               slot_of(kt) + (uint32_t)(A_BYTES + B_BYTES + h * S_BYTES + wave * 256));
      } else if constexpr (F64) {
        dma4(s_off, s_base + (2 * kt) / bpg, slot_of(kt) + (uint32_t)(A_BYTES + B_BYTES + wave * 256));
        dma4(s_off, s_base + (2 * kt + 1) / bpg, slot_of(kt) + (uint32_t)(A_BYTES + B_BYTES + S_BYTES + wave * 256));
      } else {
        dma4(s_off, s_base + kt / bpg, slot_of(kt) + (uint32_t)(A_BYTES + B_BYTES + wave * 256));
      }
    }
  };

  // ---- weight fragments of stage kt, expanded from the packed slot: column
  // n = wc*48 + 16j + l%16, K chunk c = l/16 of each 64-K step, i.e. packed
  // bytes 8c .. 8c+7 of the first (f0) and second (f1) 32-byte half of row n;
  // INT4 -> 16*q int8 in natural K order.
  const int fr_n = wc * WCOLS + (lane & 15), fr_c = lane >> 4;
  const uint32_t fr0 = (uint32_t)(fr_n * 64 + 8 * (fr_c & 1) + (((fr_c >> 1) ^ ((fr_n >> 2) & 3)) << 4));
  const uint32_t fr1 = (uint32_t)(fr_n * 64 + 8 * (fr_c & 1) + (((2 + (fr_c >> 1)) ^ ((fr_n >> 2) & 3)) << 4));
  // int8 weights: rows as the activation fragments, 16 bytes per lane
  const uint32_t fq0 = (uint32_t)lds_off(fr_n, fr_c), fq1 = (uint32_t)lds_off(fr_n, 4 + fr_c);
  // W4A16: the lane's 8 K values of column fr_n per 32-K step are 4 packed
  // bytes, at 4c of part h (swizzled by bit 3 of the row, which is bit 3 of
  // the lane), dequantized with the stage's scale of that column
  const uint32_t fw = (uint32_t)(fr_n * 32 + 4 * fr_c), fsw = (uint32_t)(((lane >> 3) & 1) << 4);
  auto load_b = [&](int kt, int j, v4i& f0, v4i& f1) {
    if constexpr (INT8W) {
      const char* pb = smem + (kt % NS) * SLOT + A_BYTES + j * 16 * kBK;
      f0 = *(const v4i*)(pb + fq0);
      f1 = *(const v4i*)(pb + fq1);
      return;
    }
    const char* pb = smem + (kt % NS) * SLOT + A_BYTES + j * 16 * 64;
    const v2u q0 = *(const v2u*)(pb + fr0);
    const v2u q1 = *(const v2u*)(pb + fr1);
    uint32_t w[8];
    if constexpr (KIL) {
      unpack8_x16_kil(q0.x, w[0], w[1]);
      unpack8_x16_kil(q0.y, w[2], w[3]);
      unpack8_x16_kil(q1.x, w[4], w[5]);
      unpack8_x16_kil(q1.y, w[6], w[7]);
    } else {
      unpack8_x16(q0.x, w[0], w[1]);
      unpack8_x16(q0.y, w[2], w[3]);
      unpack8_x16(q1.x, w[4], w[5]);
      unpack8_x16(q1.y, w[6], w[7]);
    }
    f0 = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
    f1 = v4i{(int)w[4], (int)w[5], (int)w[6], (int)w[7]};
  };

  // scales of stage kt for this lane's three columns; the MFMAs sum 16 * q
  // for packed INT4 (scaled back exactly by 1/16) and q for int8 weights
  auto read_scales = [&](int kt, int h, float* sw) {
    const float* sS = (const float*)(smem + (kt % NS) * SLOT + A_BYTES + B_BYTES + h * S_BYTES);
#pragma unroll
    for (int j = 0; j < TNB; ++j) sw[j] = sS[wc * WCOLS + 16 * j + (lane & 15)] * (INT8W ? 1.0f : 0.0625f);
  };

  // The DMAs of stage kn (the next one, or with a three-slot ring the one
  // after), issued from block row i of the stage being computed.
  auto dma_next = [&](int kn, int i) {
    if constexpr (INT8W && !GROUPED) {
      // int8 weights: the next stage's weights in block row 0 and its
      // activations in row 1, so that the last DMA has most of the stage
      // to land (spread over rows 0-6 as below: C1 40.1 against 38.4 us,
      // 4096 x 3072 x 12288 137-142 against 127-133 us)
      if (i == 0) {
#pragma unroll
        for (int c = 0; c < B_PER; ++c) dma_b(kn, c);
      } else if (i == 1) {
#pragma unroll
        for (int c = 0; c < A_PER; ++c) dma_a(kn, c);
      }
    } else {
      // scales first: issued last, their wait at the next stage showed
      // (~180 clocks per stage on the three waves that fetch them)
      if (i == 0) dma_s(kn);
      if (i < A_PER) dma_a(kn, i);
      else if (i < A_PER + B_PER) dma_b(kn, i - A_PER);
    }
  };

  // fp32 running sums (grouped) or int32 sums (per row)
  using AccT = std::conditional_t<GROUPED || DEQ, v4f, v4i>;
  AccT facc[TMB][TNB];
#pragma unroll
  for (int i = 0; i < TMB; ++i)
#pragma unroll
    for (int j = 0; j < TNB; ++j) facc[i][j] = AccT{0, 0, 0, 0};

  // One stage.  Each 16 x 16 block takes both 64-K steps back to back (the
  // second MFMA adds to the first), so its int32 group sum lives only until
  // it is folded: facc = fma(f32(acc), s_w / 16, facc).  Only the fp32 sums
  // stay resident; the group sums of two block rows are in flight, and the
  // fold of row i-1 is issued among the MFMAs of row i, whose results it does
  // not read.  A scheduling barrier per block row keeps the compiler from
  // hoisting later rows' fragment loads (registers) above it.  Fragment rows
  // 16 apart share their swizzle, so each operand and K-step needs one LDS
  // address.  The next stage's DMAs are spread over the rows.
  auto mfma_stage = [&](int kt) {
    const bool more = kt + LA < KT;  // uniform
    float sw[TNB], sw1[TNB];
    if constexpr (GROUPED) read_scales(kt, 0, sw);
    if constexpr (F64) read_scales(kt, 1, sw1);
    const char* aR0 = smem + (kt % NS) * SLOT + lds_off(wr * WROWS + (lane & 15), lane >> 4);
    const char* aR1 = smem + (kt % NS) * SLOT + lds_off(wr * WROWS + (lane & 15), 4 + (lane >> 4));
    v4i b0[TNB], b1[TNB];
#pragma unroll
    for (int j = 0; j < TNB; ++j) load_b(kt, j, b0[j], b1[j]);
    v4i n0f = *(const v4i*)aR0, n1f = *(const v4i*)aR1;
    v4i t[2][TNB], t1[F64 ? 2 : 1][TNB];
    // Empty volatile asm statements on the group sums before the fold and on
    // the fp32 sums after it pin the fold to its block row: without them the
    // compiler sinks every fold to the end of the stage and holds all 27
    // group sums at once.
    auto fold_row = [&](int i, v4i* tr, v4i* tr1) {
      if constexpr (!GROUPED) return;
#pragma unroll
      for (int j = 0; j < TNB; ++j) {
        asm volatile("" : "+v"(tr[j]));
#pragma unroll
        for (int r = 0; r < 4; ++r) facc[i][j][r] = __builtin_fmaf((float)tr[j][r], sw[j], facc[i][j][r]);
        if constexpr (F64) {
          asm volatile("" : "+v"(tr1[j]));
#pragma unroll
          for (int r = 0; r < 4; ++r) facc[i][j][r] = __builtin_fmaf((float)tr1[j][r], sw1[j], facc[i][j][r]);
        }
        asm volatile("" : "+v"(facc[i][j]));
      }
    };
#pragma unroll
    for (int i = 0; i < TMB; ++i) {
      if (i == 0 || RT::prio(i) != RT::prio(i - 1)) {
        switch (RT::prio(i)) {
          case 3: __builtin_amdgcn_s_setprio(3); break;
          case 2: __builtin_amdgcn_s_setprio(2); break;
          case 1: __builtin_amdgcn_s_setprio(1); break;
          default: __builtin_amdgcn_s_setprio(0); break;
        }
      }
      const v4i a0 = n0f, a1 = n1f;
      if (i + 1 < TMB) {
        n0f = *(const v4i*)(aR0 + (i + 1) * 16 * kBK);
        n1f = *(const v4i*)(aR1 + (i + 1) * 16 * kBK);
      }
      if constexpr (GROUPED) {
        v4i* tc = t[i & 1];
        v4i* tc1 = t1[F64 ? (i & 1) : 0];
#pragma unroll
        for (int j = 0; j < TNB; ++j) tc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0[j], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
        for (int j = 0; j < TNB; ++j) {
          if constexpr (F64) tc1[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1[j], v4i{0, 0, 0, 0}, 0, 0, 0);
          else tc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1[j], tc[j], 0, 0, 0);
        }
        if (i > 0) fold_row(i - 1, t[(i - 1) & 1], t1[F64 ? ((i - 1) & 1) : 0]);
      } else {
#pragma unroll
        for (int j = 0; j < TNB; ++j) facc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0[j], facc[i][j], 0, 0, 0);
#pragma unroll
        for (int j = 0; j < TNB; ++j) facc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1[j], facc[i][j], 0, 0, 0);
      }
      if (more) dma_next(kt + LA, i);
      __builtin_amdgcn_sched_barrier(0);
    }
    fold_row(TMB - 1, t[(TMB - 1) & 1], t1[F64 ? ((TMB - 1) & 1) : 0]);
  };

  // One W4A16 stage (DEQ), ordered (32-K half h, column block j) outer and
  // block row inner: the dequantization of fragment (h, j) + 1 is issued
  // among the MFMAs of (h, j), which do not read it, so only the first of
  // the stage's six runs with the matrix core idle (dequantizing all six
  // before the first MFMA left the MFMA pipe idle for ~100 VALU instructions
  // per wave and stage, on every wave at once after the stage barrier).
  // Each output block still takes half 0 before half 1, the stages in order:
  // the same fp32 sums as the row-outer order.  The stage's 2 x TMB activation
  // fragments stay in registers (the second half's read in the first steps).
  // Measured on MI355X against the row-outer order (both with one DMA row per
  // step): C2 4608 x 12288 x 3072 f16 332 -> 323 us, bf16 341 -> 333 us,
  // 4608 x 3072 x 12288 f16 311 -> 305 us.
  auto mfma_stage_deq = [&](int kt) {
    if constexpr (DEQ) {
      const bool more = kt + LA < KT;  // uniform
      const char* sl = smem + (kt % NS) * SLOT;
      const float* sS = (const float*)(sl + A_BYTES + B_BYTES);
      DeqScale d[TNB];
      uint32_t pk[2][TNB];
#pragma unroll
      for (int j = 0; j < TNB; ++j) {
        const char* pb = sl + A_BYTES + j * 16 * 32 + fw;
        pk[0][j] = *(const uint32_t*)(pb + fsw);
        pk[1][j] = *(const uint32_t*)(pb + (16u ^ fsw));
      }
#pragma unroll
      for (int j = 0; j < TNB; ++j) d[j] = deq_scale<OUT_DT>(sS[wc * WCOLS + 16 * j + (lane & 15)]);
      const char* aR0 = sl + lds_off(wr * WROWS + (lane & 15), lane >> 4);
      const char* aR1 = sl + lds_off(wr * WROWS + (lane & 15), 4 + (lane >> 4));
      // 192-column tiles hold both halves' activation fragments; 256-column
      // ones (144 accumulator registers) one set, each fragment re-read for
      // the second half right after its last first-half MFMA
      constexpr bool ONE_SET = RT::WIDE;
      v4i fa[2][TMB];
#pragma unroll
      for (int i = 0; i < TMB; ++i) fa[0][i] = *(const v4i*)(aR0 + i * 16 * kBK);
      auto deq_frag = [&](int q) {
        uint32_t w[4];
        deq8<OUT_DT>(pk[q / TNB][q % TNB], d[q % TNB], w);
        return v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
      };
      v4i fb[2 * TNB];
      fb[0] = deq_frag(0);
#pragma unroll
      for (int q = 0; q < 2 * TNB; ++q) {
        const int h = q / TNB, j = q % TNB;
        if (!ONE_SET && q == 1) {
#pragma unroll
          for (int i = 0; i < TMB; ++i) fa[1][i] = *(const v4i*)(aR1 + i * 16 * kBK);
        }
        if (q + 1 < 2 * TNB) fb[q + 1] = deq_frag(q + 1);
#pragma unroll
        for (int i = 0; i < TMB; ++i) {
          facc[i][j] = mfma16<OUT_DT>(fa[ONE_SET ? 0 : h][i], fb[q], facc[i][j]);
          if (ONE_SET && q == TNB - 1) fa[0][i] = *(const v4i*)(aR1 + i * 16 * kBK);
        }
        // The empty volatile asm keeps the next fragment's dequantization in
        // this step (the compiler would otherwise sink it past the DMA branch
        // below to its first use, after the next step's DMAs).  A wave issues in
        // order: two VALU instructions after each MFMA run while the matrix
        // core works on it (~17 per fragment against 9 MFMAs).
        if (q + 1 < 2 * TNB) asm volatile("" : "+v"(fb[q + 1]));
#pragma unroll
        for (int i = 0; i < TMB; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
          __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // two VALU
        }
        if (more) {
          // The next stage's DMAs.  Two-slot ring (W16): all in the first
          // two steps, scales and activations first, so that they have most
          // of the stage to land before the wait at its end (measured on
          // MI355X, against one DMA row per step: C2 4608 x 12288 x 3072
          // f16 312 -> 300 us, bf16 323 -> 309 us, 4096 x 5120 x 5120 bf16
          // 232 -> 224 us).  Three-slot ring (W16L): one DMA row per step
          // (the two-step placement measured 297 -> 303 us at
          // 4608 x 3072 x 12288 f16).
          constexpr int nd = RT::A_PER + RT::B_PER, hd = (nd + 1) / 2;
          static_assert(nd <= 2 * TNB, "DMA rows per W4A16 stage");
          if constexpr (LA == 1) {
            if (q == 0) {
#pragma unroll
              for (int r = 0; r < hd; ++r) dma_next(kt + 1, r);
            } else if (q == 1) {
#pragma unroll
              for (int r = hd; r < nd; ++r) dma_next(kt + 1, r);
            }
          } else {
            dma_next(kt + LA, q);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };

  // One stage of the 32-column fold (F32).  Per block row, the two 64-K steps
  // each run as two MFMAs on half-masked activation fragments: sums qa, qb
  // (K 0-31, 32-63 of the stage) and qc, qd (K 64-95, 96-127), folded in K
  // order.  The fold of a row's qc, qd is issued among the next row's MFMAs
  // (as in the other grouped modes), so four half sums of 16 x 16 x 3 blocks
  // are live at a time, as many as the 64-column fold holds.
  const bool lo_half = (lane >> 4) < 2;
  auto half_frag = [&](const v4i& a, bool lo) {
    const bool keep = lo ? lo_half : !lo_half;
    return v4i{keep ? a[0] : 0, keep ? a[1] : 0, keep ? a[2] : 0, keep ? a[3] : 0};
  };
  auto mfma_stage32 = [&](int kt) {
    const bool more = kt + 1 < KT;  // uniform
    float s0[TNB], s1[TNB], s2[TNB], s3[TNB];
    read_scales(kt, 0, s0);
    read_scales(kt, 1, s1);
    read_scales(kt, 2, s2);
    read_scales(kt, 3, s3);
    const char* aR0 = smem + (kt % NS) * SLOT + lds_off(wr * WROWS + (lane & 15), lane >> 4);
    const char* aR1 = smem + (kt % NS) * SLOT + lds_off(wr * WROWS + (lane & 15), 4 + (lane >> 4));
    v4i b0[TNB], b1[TNB];
#pragma unroll
    for (int j = 0; j < TNB; ++j) load_b(kt, j, b0[j], b1[j]);
    v4i n0f = *(const v4i*)aR0, n1f = *(const v4i*)aR1;
    v4i qa[TNB], qb[TNB], qc[TNB], qd[TNB];
    auto fold2 = [&](int i, v4i* x, v4i* y, const float* sx, const float* sy) {
#pragma unroll
      for (int j = 0; j < TNB; ++j) {
        asm volatile("" : "+v"(x[j]));
#pragma unroll
        for (int r = 0; r < 4; ++r) facc[i][j][r] = __builtin_fmaf((float)x[j][r], sx[j], facc[i][j][r]);
        asm volatile("" : "+v"(y[j]));
#pragma unroll
        for (int r = 0; r < 4; ++r) facc[i][j][r] = __builtin_fmaf((float)y[j][r], sy[j], facc[i][j][r]);
        asm volatile("" : "+v"(facc[i][j]));
      }
    };
#pragma unroll
    for (int i = 0; i < TMB; ++i) {
      if (i == 0 || RT::prio(i) != RT::prio(i - 1)) {
        switch (RT::prio(i)) {
          case 3: __builtin_amdgcn_s_setprio(3); break;
          case 2: __builtin_amdgcn_s_setprio(2); break;
          case 1: __builtin_amdgcn_s_setprio(1); break;
          default: __builtin_amdgcn_s_setprio(0); break;
        }
      }
      const v4i a0 = n0f, a1 = n1f;
      if (i + 1 < TMB) {
        n0f = *(const v4i*)(aR0 + (i + 1) * 16 * kBK);
        n1f = *(const v4i*)(aR1 + (i + 1) * 16 * kBK);
      }
      const v4i a0l = half_frag(a0, true), a0h = half_frag(a0, false);
#pragma unroll
      for (int j = 0; j < TNB; ++j) qa[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0l, b0[j], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
      for (int j = 0; j < TNB; ++j) qb[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0h, b0[j], v4i{0, 0, 0, 0}, 0, 0, 0);
      if (i > 0) fold2(i - 1, qc, qd, s2, s3);
      const v4i a1l = half_frag(a1, true), a1h = half_frag(a1, false);
#pragma unroll
      for (int j = 0; j < TNB; ++j) qc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1l, b1[j], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
      for (int j = 0; j < TNB; ++j) qd[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1h, b1[j], v4i{0, 0, 0, 0}, 0, 0, 0);
      fold2(i, qa, qb, s0, s1);
      if (more) dma_next(kt + 1, i);
      __builtin_amdgcn_sched_barrier(0);
    }
    fold2(TMB - 1, qc, qd, s2, s3);
  };

  // Int8 weights: the last block row's MFMAs of each stage are issued after
  // the next stage's barrier, behind that stage's first fragment reads, so the
  // MFMA pipes have work while those reads are in flight.  Their operands stay
  // in registers: the activation row in pa0 / pa1, the weight fragments in
  // the set the stage loaded (two sets, alternating by stage).  4096 x 3072 x
  // 12288: 133-137 against 125-130 us; C1 38.4 against 38.1 us.  With INT4
  // weights (expanded in registers) the same order was 1-4 % slower.
  v4i pa0, pa1;
  auto row_mfma = [&](int i, const v4i& a0, const v4i& a1, const v4i* b0, const v4i* b1) {
#pragma unroll
    for (int j = 0; j < TNB; ++j) facc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0[j], facc[i][j], 0, 0, 0);
#pragma unroll
    for (int j = 0; j < TNB; ++j) facc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1[j], facc[i][j], 0, 0, 0);
  };
  auto row_stage = [&](int kt, v4i* b0, v4i* b1, const v4i* pb0, const v4i* pb1) {
    const bool more = kt + 1 < KT;  // uniform
    const char* aR0 = smem + (kt % NS) * SLOT + lds_off(wr * WROWS + (lane & 15), lane >> 4);
    const char* aR1 = smem + (kt % NS) * SLOT + lds_off(wr * WROWS + (lane & 15), 4 + (lane >> 4));
#pragma unroll
    for (int j = 0; j < TNB; ++j) load_b(kt, j, b0[j], b1[j]);
    v4i n0f = *(const v4i*)aR0, n1f = *(const v4i*)aR1;
    __builtin_amdgcn_s_setprio(3);
    if (kt > 0) row_mfma(TMB - 1, pa0, pa1, pb0, pb1);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < TMB - 1; ++i) {
      if (i > 0 && RT::prio(i) != RT::prio(i - 1)) {
        switch (RT::prio(i)) {
          case 2: __builtin_amdgcn_s_setprio(2); break;
          case 1: __builtin_amdgcn_s_setprio(1); break;
          default: __builtin_amdgcn_s_setprio(0); break;
        }
      }
      const v4i a0 = n0f, a1 = n1f;
      n0f = *(const v4i*)(aR0 + (i + 1) * 16 * kBK);
      n1f = *(const v4i*)(aR1 + (i + 1) * 16 * kBK);
      row_mfma(i, a0, a1, b0, b1);
      if (more) dma_next(kt + 1, i);
      __builtin_amdgcn_sched_barrier(0);
    }
    pa0 = n0f;
    pa1 = n1f;
  };

  // ---- prologue: stages 0 .. LA-1 in flight
  for (int s0 = 0; s0 < LA && s0 < KT; ++s0) {
#pragma unroll
    for (int c = 0; c < A_PER; ++c) dma_a(s0, c);
#pragma unroll
    for (int c = 0; c < B_PER; ++c) dma_b(s0, c);
    dma_s(s0);
  }
  // this wave's DMA instructions per stage (wave-uniform): with two stages in
  // flight, stage s has landed once no more than those of stage s+1 remain
  // outstanding (they retire in issue order)
  int per_stage = (SCALED && s_wave) ? RT::NSC : 0;
#pragma unroll
  for (int c = 0; c < A_PER; ++c) per_stage += wave + 8 * c < A_BLOCKS;
#pragma unroll
  for (int c = 0; c < B_PER; ++c) per_stage += wave + 8 * c < B_BLOCKS;
  auto wait_stage = [&](int s) {
    if (LA == 1 || s + 1 >= KT) {
      wait_vm<0>();
      return;
    }
    switch (per_stage) {
      case 0: wait_vm<0>(); break;
      case 1: wait_vm<1>(); break;
      case 2: wait_vm<2>(); break;
      case 3: wait_vm<3>(); break;
      case 4: wait_vm<4>(); break;
      case 5: wait_vm<5>(); break;
      case 6: wait_vm<6>(); break;
      case 7: wait_vm<7>(); break;
      default: wait_vm<0>(); break;
    }
  };

  if constexpr (!INT8W || GROUPED) {
    for (int s = 0; s < KT; ++s) {
      wait_stage(s);
      lds_barrier();  // stage s resident; every wave is done with stage s-1
      if constexpr (F32) mfma_stage32(s);
      else if constexpr (DEQ) mfma_stage_deq(s);
      else mfma_stage(s);
    }
  } else {
    v4i bA0[TNB], bA1[TNB], bB0[TNB], bB1[TNB];
    for (int s = 0; s < KT; s += 2) {
      wait_vm<0>();
      lds_barrier();
      row_stage(s, bA0, bA1, bB0, bB1);
      if (s + 1 < KT) {
        wait_vm<0>();
        lds_barrier();
        row_stage(s + 1, bB0, bB1, bA0, bA1);
      }
    }
    __builtin_amdgcn_s_setprio(0);
    if ((KT - 1) & 1) row_mfma(TMB - 1, pa0, pa1, bB0, bB1);
    else row_mfma(TMB - 1, pa0, pa1, bA0, bA1);
  }

  // ---- epilogue: finish in registers, stage the tile through LDS row-major,
  // write whole rows with 16-byte stores (the host picks this kernel only for
  // 16-byte aligned outputs and residuals).
  constexpr int RS = EPI_RS;
  constexpr int CPR = BN / 8;
  lds_barrier();
  u16* ot = (u16*)smem;
  float* sa_l = (float*)(smem + BM * RS * 2);
  float* b_l = sa_l + BM;
  float* sw_l = b_l + BN;
  bool res_lds = false;
  if constexpr (EPI) {
    res_lds = epi.res != nullptr;
    if (res_lds) {
      for (int c = tid; c < BM * CPR; c += kNT) {
        const int row = c / CPR, col = (c % CPR) * 8;
        const int m = m0 + row, n = n0 + col;
        if (m < M && n < N)
          *(v4u*)(ot + row * RS + col) = *(const v4u*)((const u16*)epi.res + (int64_t)m * epi.ldr + n);
      }
    }
  }
  if (tid < BM) sa_l[tid] = pre_sa;
  if (tid < BN) {
    b_l[tid] = pre_b;
    sw_l[tid] = pre_sw;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < TNB; ++j) {
    const int nl = wc * WCOLS + 16 * j + (lane & 15);
    const float b = b_l[nl];
    const float sw = sw_l[nl];
#pragma unroll
    for (int i = 0; i < TMB; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int ml = wr * WROWS + 16 * i + 4 * (lane >> 4) + r;
        float v;
        if constexpr (GROUPED) {
          v = facc[i][j][r] * sa_l[ml];
        } else if constexpr (DEQ) {
          v = facc[i][j][r];
        } else {
          float a = (float)facc[i][j][r];
          if constexpr (!INT8W) a *= 0.0625f;
          v = a * (sa_l[ml] * sw);
        }
        if (bias != nullptr) v = v + b;
        if constexpr (EPI) {
          v = epi_act(v, epi.act);
          if (res_lds) {
            const u16 rv = ot[ml * RS + nl];
            v = v + (epi.res_dt == IC_DTYPE_F16 ? f16_to_f32(rv) : bf16_to_f32(rv));
          }
        }
        u16 h;
        if constexpr (OUT_DT == IC_DTYPE_F16) h = f32_to_f16(v);
        else h = f32_to_bf16(v);
        ot[ml * RS + nl] = h;
      }
      if constexpr (EPI) __builtin_amdgcn_sched_barrier(0);
    }
  }
  __syncthreads();
#pragma unroll 4
  for (int c = tid; c < BM * CPR; c += kNT) {
    const int row = c / CPR, col = (c % CPR) * 8;
    const int m = m0 + row, n = n0 + col;
    if (m < M && n < N) *(v4u*)((u16*)C + (int64_t)m * ldc + n) = *(const v4u*)(ot + row * RS + col);
  }
}

}  // namespace
