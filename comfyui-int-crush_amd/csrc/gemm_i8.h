// INT8 x INT8 -> INT32 MFMA GEMM with fused dequant epilogue (gfx950).
//
//   out[m, n] = f32(acc[m, n]) * (s_a[m] * s_w[n]) + bias[n]                (per-row weight scale)
//   out[m, n] = (sum_g f32(acc_g[m, n]) * s_w[n, g]) * s_a[m] + bias[n]     (per-group weight scale)
//
// A = activation codes [M, K] int8, K-major.  B = weights [N, K], K-major, as
// int8 (W8A8, triton_int8_gemm.py:46-132) or as packed INT4 nibbles (W4A8,
// triton_w4a8_gemm.py:40-108 plus the unpack of triton_int4_to_int8_unpack.py:26-52,
// here fused into the weight staging so the unpacked weight never reaches HBM).
//
// Work decomposition (one 512-thread workgroup per CU, two waves per SIMD):
//   * a BM x BN output tile per workgroup, 8 waves in a WGM x (8/WGM) grid, each
//     wave owning (BM/WGM) x (BN*WGM/8) built from v_mfma_i32_32x32x32_i8 tiles
//     whose int32 accumulators stay in architectural VGPRs;
//   * K advances 128 bytes per stage (one 128-wide scale group) through an
//     NS-deep LDS ring.  Every global read of the main loop -- activation
//     rows, int8 or packed INT4 weight rows, per-group scales -- is a direct
//     global->LDS DMA (global_load_lds) issued from inline assembly, so no
//     VGPR holds staged data and the only memory waits are the explicit,
//     static vmcnt waits of the pipeline (the compiler cannot see these DMAs
//     and so does not serialise LDS accesses behind them).  A stage's DMAs
//     are issued in slices between the MFMA K-steps of the stage before, so
//     no wave stalls at a burst of DMA issues before its MFMAs;
//   * activation and int8 weight chunks land XOR-swizzled by row (the issuing
//     lane picks the global chunk), so the ds_read_b128 fragment loads are
//     bank-conflict free;
//   * packed INT4 weights are expanded once per workgroup and stage from the
//     ring into an LDS tile as 16*q (int8): two masks and a byte permute per
//     8 nibbles; the factor 16 is removed exactly in the epilogue;
//   * per-group scales (group 128 = one stage) fold the int32 partials into an
//     fp32 accumulator with one convert + FMA per element and group; two int32
//     accumulator sets alternate between groups so the fold of group g runs
//     while the MFMAs of group g+1 execute.
#pragma once
#include <type_traits>

#include "gemm_common.h"
#include "gemm_i8_big.h"
#include "rq_common.h"

namespace ic_gemm {
struct GemmArgs {
  const int8_t* A; int64_t lda; const uint8_t* B; int64_t ldb;
  const float* s_a; const float* s_w; int G;
  const void* bias; int bias_dt; void* C; int out_dt; int64_t ldc; int M, N, K;
  int32_t* acc_out; bool int4;
  void* ws = nullptr; int64_t ws_bytes = 0;  // split-K workspace (optional)
  ic_epi epi{};                              // activation / residual epilogue
  bool kil = false;                          // packed INT4 in the K-interleaved nibble order
};
}  // namespace ic_gemm

// GEMM launches with the activation / residual epilogue compiled in
// (gemm_i8_epi.hip).
int ic_gemm_run_epi(const ic_gemm::GemmArgs& g, hipStream_t st, const char* who, bool force_generic);
// gemm_i8_big_kernel on packed INT4 in the K-interleaved nibble order, for
// weight mode `mode` (gemm_i8_kil.hip; its own translation unit, so that
// these instantiations compile in parallel with the others).
hipError_t ic_launch_big_kil(const ic_gemm::GemmArgs& g, int out_dt, bool epi, int mode, hipStream_t st);

namespace {
using ic_gemm::GemmArgs;

// Tile configuration: BM x BN output tile, WGM wave rows, NS-deep LDS ring.
template <int BM_, int BN_, int WGM_, int NS_, bool INT4_, int GS_>
struct Tile {
  static constexpr int BM = BM_, BN = BN_, WGM = WGM_, NS = NS_;
  static constexpr bool INT4 = INT4_;
  static constexpr int GS = GS_;
  static constexpr int A_BYTES = BM * kBK;
  static constexpr int B_BYTES = INT4 ? BN * kBK / 2 : BN * kBK;  // packed for INT4
  static constexpr int S_BYTES = GS ? BN * 4 : 0;
  static constexpr int SLOT = A_BYTES + B_BYTES + S_BYTES;
  static constexpr int BU_BYTES = INT4 ? BN * kBK : 0;  // one unpacked INT4 tile
  static constexpr int EPI_RS = BN + 8;  // 16-bit output staging row stride (elements)
  static constexpr size_t epi_bytes() { return (size_t)BM * EPI_RS * 2 + (size_t)(BM + 2 * BN) * 4; }
  static constexpr size_t ring_bytes() { return (size_t)NS * SLOT + (size_t)BU_BYTES; }
  static constexpr size_t lds_bytes() { return ring_bytes() > epi_bytes() ? ring_bytes() : epi_bytes(); }
  // chained epilogue (ROT): the staging tile and its scale rows, the SmoothRot
  // reciprocals of the tile's columns, then every wave's fp64 exchange slice
  static constexpr size_t chain_xoff() { return (epi_bytes() + (size_t)BN * 4 + 15) / 16 * 16; }
  static constexpr size_t chain_bytes() { return chain_xoff() + (size_t)rq::xbuf_doubles<kNT * 16>() * 8; }
  static constexpr size_t chain_lds_bytes() { return ring_bytes() > chain_bytes() ? ring_bytes() : chain_bytes(); }
};

// PART (split-K): workgroup (x, y) computes tile x over the K stages of
// slice y of gridDim.y and writes its 4-byte partials -- the int32 sum
// (per-row scales) or the fp32 group fold (grouped) -- to
// acc_out[(y * M + m) * N + n]; splitk_reduce_kernel finishes them.
//
// ROT (2, 3, 4; with EPI and a 16-bit output): the chained MLP epilogue of
// ic_gemm_*_chain.  Each finished tile of h = RN_dt(epilogue value) is
// prepared, in LDS, as the next linear's activation -- SmoothRot divide and
// R = 4^ROT block Hadamard, the first half of _prep_activation -- before it
// is stored.
template <class TL, int OUT_DT, bool ACC_OUT, bool PART = false, bool EPI = false, int ROT = 0>
__global__ __launch_bounds__(kNT, 1) void gemm_i8_kernel(
    const int8_t* __restrict__ A, int64_t lda, const uint8_t* __restrict__ B, int64_t ldb,
    const float* __restrict__ s_a, const float* __restrict__ s_w, int G,
    const void* __restrict__ bias, int bias_dt, void* __restrict__ C, int64_t ldc, int M, int N,
    int K, int32_t* __restrict__ acc_out, ic_epi epi, W4Sel wsel) {
  constexpr int BM = TL::BM, BN = TL::BN, WGM = TL::WGM, NS = TL::NS, GS = TL::GS;
  constexpr bool INT4 = TL::INT4;
  constexpr int WGN = 8 / WGM;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int A_DMA = BM / 64;                  // 1 KB DMA blocks of A per wave per stage
  constexpr int B_DMA = INT4 ? BN / 128 : BN / 64;  // same for (packed) weights
  constexpr int S_WAVES = GS ? BN / 64 : 0;       // waves issuing one scale DMA per stage
  constexpr int D = A_DMA + B_DMA;
  constexpr int PK = INT4 ? BN * (kBK / 2) / kNT : 0;  // packed weight bytes unpacked per thread
  static_assert(TM >= 1 && TN >= 1 && A_DMA >= 1 && B_DMA >= 1, "tile too small");
  static_assert(!INT4 || PK == 16 || PK == 32, "INT4 unpack split");
  static_assert(GS == 0 || GS == 128, "group size");
  static_assert(NS >= 2 && S_WAVES <= 8, "ring depth");

  extern __shared__ __attribute__((aligned(16))) char smem[];
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_char*)smem;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = wave / WGN, wc = wave % WGN;
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int tm, tn;
  tile_coords(blockIdx.x, tiles_m * tiles_n, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  // Operands of the staged 16-bit epilogue (activation scale of row m0 + tid,
  // bias and per-row weight scale of column n0 + tid), loaded now so that
  // their latency passes under the main loop instead of after it.
  static_assert(BM <= kNT && BN <= kNT, "one epilogue operand per thread");
  float pre_sa = 0.0f, pre_b = 0.0f, pre_sw = 0.0f;
  if constexpr (OUT_DT != IC_DTYPE_F32 && !PART) {
    if (C != nullptr) {
      if (tid < BM) pre_sa = s_a[min(m0 + tid, M - 1)];
      if (tid < BN) {
        const int n = min(n0 + tid, N - 1);
        if (bias != nullptr) pre_b = ld_any_f32(bias, bias_dt, n);
        if constexpr (GS == 0) pre_sw = s_w[n];
      }
    }
  }
  const int KT_all = K / kBK;
  const int kt0 = PART ? (int)((int64_t)blockIdx.y * KT_all / gridDim.y) : 0;
  const int KT = PART ? (int)((int64_t)(blockIdx.y + 1) * KT_all / gridDim.y) - kt0 : KT_all;
  const bool s_wave = wave < S_WAVES;

  // ---- DMA addressing.  A / int8 B: lane L of a 1 KB block covers LDS row
  // 8*blk + L/8, chunk slot L%8, and loads global chunk (L%8) ^ swz(row).
  // Packed B: 16 rows of 64 bytes per block, unswizzled.  Scales: one dword
  // per lane, column n0 + 64*wave + lane of group kt.
  const int dma_row = lane >> 3;
  uint32_t a_off[A_DMA];
#pragma unroll
  for (int c = 0; c < A_DMA; ++c) {
    const int row = 8 * (wave + 8 * c) + dma_row;
    a_off[c] = (uint32_t)(min(row, M - 1 - m0) * lda + (((lane & 7) ^ swz(row)) << 4));
  }
  uint32_t b_off[B_DMA];
#pragma unroll
  for (int c = 0; c < B_DMA; ++c) {
    if constexpr (INT4) {
      const int row = 16 * (wave + 8 * c) + (lane >> 2);
      b_off[c] = (uint32_t)(min(row, N - 1 - n0) * ldb + ((lane & 3) << 4));
    } else {
      const int row = 8 * (wave + 8 * c) + dma_row;
      b_off[c] = (uint32_t)(min(row, N - 1 - n0) * ldb + (((lane & 7) ^ swz(row)) << 4));
    }
  }
  const uint32_t s_off = GS ? (uint32_t)(min(64 * wave + lane, N - 1 - n0) * G * 4) : 0u;
  const int8_t* a_base = A + (int64_t)m0 * lda + (int64_t)kt0 * kBK;
  const uint8_t* b_base = B + (int64_t)n0 * ldb + (int64_t)kt0 * (INT4 ? kBK / 2 : kBK);
  const float* s_base = GS ? s_w + (int64_t)n0 * G : nullptr;
  // scale groups of 128 * spg columns: stage kt0 + kt folds with group (kt0 + kt) / spg
  const int spg = GS ? (K / G) / kBK : 1;

  // The D DMA instructions of one stage are issued in kParts slices, one per
  // K-step of the MFMA loop: a wave that issued a whole stage at once stalled
  // at issue instead of starting its MFMAs.  Slice p holds the blocks d with
  // d % kParts == p (A blocks first, then B); the scale DMA goes last.
  //
  // kt may run past the end of K (per-row-scale kernels, below): the slot is
  // still kt % NS, the one the current step frees, and only the source is
  // clamped to the last stage, so a redundant reload never lands in a slot
  // that a later step reads.
  constexpr int kParts = kBK / 32;
  constexpr bool kFullSteps = GS == 0;  // see below
  auto issue_dma_part = [&](int kt_slot, int part) {
    const uint32_t slot = lds0 + (uint32_t)((kt_slot % NS) * TL::SLOT);
    // (the exact-issue kernels never pass kt_slot >= KT)
    const int kt = kFullSteps ? __builtin_amdgcn_readfirstlane(min(kt_slot, KT - 1)) : kt_slot;
    const int8_t* ab = a_base + (int64_t)kt * kBK;
#pragma unroll
    for (int c = 0; c < A_DMA; ++c)
      if (c % kParts == part) dma16(a_off[c], ab, slot + (uint32_t)((wave + 8 * c) * 1024));
    const uint8_t* bb = b_base + (int64_t)kt * (INT4 ? kBK / 2 : kBK);
#pragma unroll
    for (int c = 0; c < B_DMA; ++c)
      if ((A_DMA + c) % kParts == part) dma16(b_off[c], bb, slot + (uint32_t)(TL::A_BYTES + (wave + 8 * c) * 1024));
    if constexpr (GS != 0) {
      if (part == kParts - 1 && s_wave)
        dma4(s_off, s_base + (kt0 + kt) / spg, slot + (uint32_t)(TL::A_BYTES + TL::B_BYTES + wave * 256));
    }
  };
  auto issue_dma = [&](int kt) {
#pragma unroll
    for (int p = 0; p < kParts; ++p) issue_dma_part(kt, p);
  };
  // Per-row-scale kernels issue a full stage on every step: past the end of K
  // a redundant reload of the last stage's bytes into the slot the step frees,
  // which nothing reads.  The step then has no branch around its DMA issue, so the
  // compiler schedules the next K-step's LDS reads among this one's MFMAs
  // (4-6 % faster W8A8; the grouped kernels, VALU-bound, gained nothing and
  // keep the exact issue).  The trailing reloads are drained before the
  // epilogue reuses LDS.
  // Top of step s: stages s+1 .. s+NS-2 may stay in flight (D DMA
  // instructions each, one more on the waves that also fetch scales); near the
  // end of K (exact issue), wait for everything.
  auto wait_stage = [&](int s) {
    if constexpr (kFullSteps) {
      if (s_wave) wait_vm<(D + 1) * (NS - 2)>();
      else wait_vm<D * (NS - 2)>();
      return;
    }
    if constexpr (NS > 2) {
      if (s + NS - 2 < KT) {
        if (s_wave) wait_vm<(D + 1) * (NS - 2)>();
        else wait_vm<D * (NS - 2)>();
        return;
      }
    }
    wait_vm<0>();
  };

  // ---- packed INT4 -> 16*q int8 tile in LDS (either nibble order: wsel).
  // One buffer suffices: the barrier at the top of each step orders the MFMA
  // reads of step s-1 before the unpack of step s.
  auto unpack = [&](int kt) {
    if constexpr (INT4) {
      const char* bp = smem + (kt % NS) * TL::SLOT + TL::A_BYTES;
      char* bu = smem + NS * TL::SLOT;
#pragma unroll
      for (int h = 0; h < PK / 16; ++h) {
        const int idx = tid + kNT * h;      // 16-byte packed chunk index
        const int row = idx >> 2, part = idx & 3;
        const v4u p = *(const v4u*)(bp + idx * 16);
        uint32_t w[8];
        unpack8_x16(p.x, w[0], w[1], wsel);
        unpack8_x16(p.y, w[2], w[3], wsel);
        unpack8_x16(p.z, w[4], w[5], wsel);
        unpack8_x16(p.w, w[6], w[7], wsel);
        *(v4u*)(bu + lds_off(row, 2 * part)) = v4u{w[0], w[1], w[2], w[3]};
        *(v4u*)(bu + lds_off(row, 2 * part + 1)) = v4u{w[4], w[5], w[6], w[7]};
      }
    }
  };

  typedef int v4i_t __attribute__((ext_vector_type(4)));
  constexpr bool kPingPong = GS == 128 && TM * TN <= 2 * 2;
  constexpr int NSET = kPingPong ? 2 : 1;
  v16i acc[NSET][TM][TN];
  v16f facc[GS == 128 ? TM : 1][GS == 128 ? TN : 1];
#pragma unroll
  for (int s = 0; s < NSET; ++s)
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[s][i][j] = v16i{};
  if constexpr (GS == 128) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) facc[i][j] = v16f{};
  }

  auto out_row = [&](int i, int r) { return m0 + wr * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); };
  auto out_col = [&](int j) { return n0 + wc * WN + j * 32 + (lane & 31); };

  // Chained prep of a staged tile (ROT): ot holds h = RN_dt(epilogue value)
  // row-major with row stride BN + 8.  In passes of 8192 positions each lane
  // takes 16 consecutive columns of one row and, exactly as the fast prep
  // kernel does, divides them by the SmoothRot factors (RN_dt(RN32(h * rcp))
  // where that product is a normal DT value, the IEEE quotient otherwise),
  // applies the bf16 flush rule, runs the radix-4 digits in fp64 (digits 0-1
  // in registers, 2-3 through this wave's exchange slice), rounds once to DT
  // and writes the rotated values back in place.  A block of R columns never
  // straddles tiles (R divides BN), so each block is whole in one lane group.
  auto chain_rotate = [&](u16* ot, const float* rc_l, double* xb) {
    if constexpr (ROT != 0) {
      static_assert(EPI && !ACC_OUT && !PART && OUT_DT != IC_DTYPE_F32, "chained epilogue configuration");
      static_assert(BN == 256 && ROT >= 2 && ROT <= 4, "chained rotation tiles");
      constexpr int RS = TL::EPI_RS;
      constexpr int RC = ROT <= 2 ? 0 : 1;
      constexpr int kPass = BM * BN / (kNT * 16);
      const bool has_sr = epi.sr_rcp != nullptr;
      for (int ps = 0; ps < kPass; ++ps) {
        const int p0 = ps * (kNT * 16) + 16 * tid;
        const int row = p0 / BN, col = p0 % BN;
        const v4u ha = *(const v4u*)(ot + row * RS + col);
        const v4u hb = *(const v4u*)(ot + row * RS + col + 8);
        const uint32_t hw[8] = {ha.x, ha.y, ha.z, ha.w, hb.x, hb.y, hb.z, hb.w};
        float xs[16];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          xs[2 * i] = rq::bits16_f32<OUT_DT>((u16)(hw[i] & 0xffffu));
          xs[2 * i + 1] = rq::bits16_f32<OUT_DT>((u16)(hw[i] >> 16));
        }
        rq::Bf16RunStats fst{0u, 0.0f};
        bool fst_ok = false;
        if (has_sr) {
          float rc[16], xo[16];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const v4f r = *(const v4f*)(rc_l + col + 4 * i);
            rc[4 * i] = r.x; rc[4 * i + 1] = r.y; rc[4 * i + 2] = r.z; rc[4 * i + 3] = r.w;
          }
          float hmin = __builtin_huge_valf();
          uint32_t hmax_bits = 0u;
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            xo[j] = xs[j];
            xs[j] = round_to_dt<OUT_DT>(xs[j] * rc[j]);
            hmin = __builtin_fminf(hmin, __builtin_fabsf(xs[j]));
            if constexpr (OUT_DT == IC_DTYPE_BF16) {
              const uint32_t a = __float_as_uint(xs[j]) & 0x7fffffffu;
              hmax_bits = hmax_bits > a ? hmax_bits : a;
            }
          }
          const bool nonfinite = OUT_DT == IC_DTYPE_BF16 && hmax_bits >= 0x7f800000u;
          fst = rq::Bf16RunStats{hmax_bits, hmin};
          fst_ok = true;
          if (__builtin_expect(!(hmin > dt_min_normal<OUT_DT>()) || nonfinite, 0)) {
            fst_ok = false;
            // columns of a partial last tile read a valid factor and are never stored
            const int kc = min(n0 + col, N - 16);
#pragma unroll
            for (int j = 0; j < 16; ++j) xs[j] = div_round_dt<OUT_DT>(xo[j], rc[j], epi.sr_f, kc + j);
          }
        }
        if constexpr (OUT_DT == IC_DTYPE_BF16) {
          if (!fst_ok) fst = rq::bf16_run_stats(xs);
          rq::bf16_flush_small<ROT, kNT>(xs, nullptr, fst);
        }
        double v[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = (double)xs[j];
        rq::stage_lo(v);
        rq::stage_hi(v);
        if constexpr (ROT >= 3) {
#pragma unroll
          for (int j = 0; j < 16; ++j) xb[rq::xslot(16 * tid + j)] = v[j];
          __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
          __builtin_amdgcn_wave_barrier();
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
          const int g = tid >> 4, l = tid & 15;
#pragma unroll
          for (int h = 0; h < 16; ++h) v[h] = xb[rq::xslot(256 * g + 16 * h + l)];
          rq::stage_lo(v);
          if constexpr (ROT >= 4) rq::stage_hi(v);
          // every lane has read its slots before the next pass rewrites them
          __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
          __builtin_amdgcn_wave_barrier();
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int p = ps * (kNT * 16) + rq::tile_pos<RC>(tid, j);
          ot[(p / BN) * RS + p % BN] = rq::f32_bits16<OUT_DT>(round_f64_to_dt<OUT_DT>(v[j]));
        }
      }
    }
  };

  // Scales of group kt for this lane's columns, from the stage's LDS slot.
  auto read_scales = [&](int kt, float* sw) {
    if constexpr (GS == 128) {
      const float* sS = (const float*)(smem + (kt % NS) * TL::SLOT + TL::A_BYTES + TL::B_BYTES);
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        sw[j] = sS[wc * WN + j * 32 + (lane & 31)];
        if constexpr (INT4) sw[j] *= 0.0625f;  // acc holds 16 * the true sum
      }
    }
  };

  // Fold of one 32x32 tile t of accumulator set FS (group g) into facc:
  // facc += f32(acc_g) * s_w[n, g] (16 converts + 16 FMAs per lane).
  auto fold_tile = [&](int g, auto fs_c, int t, const float* sw) {
    constexpr int FS = decltype(fs_c)::value;
    const int i = t / TN, j = t % TN;
    // Anchors: empty volatile asm statements on the tile before and on its
    // fp32 accumulator after the fold keep the register-only fold between the
    // stage's barriers (volatile asm stays ordered), so it can neither be
    // hoisted nor sunk out of the MFMA region it is interleaved with.
    asm volatile("" : "+v"(acc[FS][i][j]));
    if constexpr (ACC_OUT) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = out_row(i, r), nn = out_col(j);
        if (m < M && nn < N)
          acc_out[((int64_t)g * M + m) * N + nn] = INT4 ? (acc[FS][i][j][r] >> 4) : acc[FS][i][j][r];
      }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) facc[i][j][r] = __builtin_fmaf((float)acc[FS][i][j][r], sw[j], facc[i][j][r]);
    asm volatile("" : "+v"(facc[i][j]));  // nor sunk past the next barrier
  };
  auto fold = [&](int g, auto fs_c, const float* sw) {
#pragma unroll
    for (int t = 0; t < TM * TN; ++t) fold_tile(g, fs_c, t, sw);
  };

  // One stage (4 K-steps of 32) into accumulator set SET; ZF starts the set
  // afresh (MFMA with a zero addend) on the first K-step.  With FOLD, the fold
  // of the previous group (set FS, scales sw_f) is spread over the stage, one
  // 32x32 tile per K-step, between the MFMAs of the other accumulator set.
  auto mfma_stage = [&](int kt, int dma_kt, auto set_c, auto zero_c, auto fold_c, auto fs_c, int g_f,
                        const float* sw_f) {
    constexpr int SET = decltype(set_c)::value;
    constexpr bool ZF = decltype(zero_c)::value;
    constexpr bool FOLD = decltype(fold_c)::value;
    const char* sA = smem + (kt % NS) * TL::SLOT;
    const char* sB = INT4 ? smem + NS * TL::SLOT : sA + TL::A_BYTES;
#pragma unroll
    for (int ks = 0; ks < kBK / 32; ++ks) {
      v4i_t a[TM], b[TN];
      const int ch = 2 * ks + (lane >> 5);
#pragma unroll
      for (int i = 0; i < TM; ++i) a[i] = *(const v4i_t*)(sA + lds_off(wr * WM + i * 32 + (lane & 31), ch));
#pragma unroll
      for (int j = 0; j < TN; ++j) b[j] = *(const v4i_t*)(sB + lds_off(wc * WN + j * 32 + (lane & 31), ch));
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          if (ZF && ks == 0) acc[SET][i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], v16i{}, 0, 0, 0);
          else acc[SET][i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], acc[SET][i][j], 0, 0, 0);
        }
      if constexpr (kFullSteps) issue_dma_part(dma_kt, ks);
      else if (dma_kt < KT) issue_dma_part(dma_kt, ks);
      // The fold's instructions are placed among this K-step's MFMAs by the
      // compiler; fixed MFMA:VALU interleave patterns measured 3-5 % slower.
      if constexpr (FOLD) {
        if (ks < TM * TN) fold_tile(g_f, fs_c, ks, sw_f);
      }
    }
    if constexpr (FOLD && TM * TN > kBK / 32) {
#pragma unroll
      for (int t = kBK / 32; t < TM * TN; ++t) fold_tile(g_f, fs_c, t, sw_f);
    }
  };

  // ---- prologue: NS-1 stages in flight
#pragma unroll
  for (int t = 0; t < NS - 1; ++t)
    if constexpr (kFullSteps) issue_dma(t);
    else if (t < KT) issue_dma(t);

  // One pipeline step: make stage s resident (this wave's DMAs, then the
  // barrier for everyone's), expand packed weights (second barrier), then run
  // the MFMAs of stage s while refilling the ring slot freed by step s-1.
  using T0 = std::integral_constant<int, 0>;
  using T1 = std::integral_constant<int, 1>;
  using ZF = std::true_type;
  using NZ = std::false_type;
  float sw_a[TN], sw_b[TN];
  auto step = [&](int s, auto set_c, auto zero_c, float* sw_read, auto fold_c, auto fs_c, int g_f,
                  const float* sw_f) {
    wait_stage(s);
    lds_barrier();
    if constexpr (INT4) {
      unpack(s);
      lds_barrier();
    }
    read_scales(s, sw_read);
    // keep the (register-only) fold inside the MFMA region instead of letting
    // it be hoisted above the barriers
    __builtin_amdgcn_sched_barrier(0);
    mfma_stage(s, s + NS - 1, set_c, zero_c, fold_c, fs_c, g_f, sw_f);
    __builtin_amdgcn_sched_barrier(0);
  };

  if constexpr (GS == 0) {
    for (int s = 0; s < KT; ++s) step(s, T0{}, NZ{}, sw_a, NZ{}, T0{}, 0, sw_a);
  } else if constexpr (kPingPong) {
    // set g&1 accumulates group g while set (g-1)&1 (group g-1) is folded
    step(0, T0{}, ZF{}, sw_a, NZ{}, T1{}, 0, sw_b);
    int g = 1;
    for (; g + 1 < KT; g += 2) {
      step(g, T1{}, ZF{}, sw_b, ZF{}, T0{}, g - 1, sw_a);
      step(g + 1, T0{}, ZF{}, sw_a, ZF{}, T1{}, g, sw_b);
    }
    if (g < KT) {
      step(g, T1{}, ZF{}, sw_b, ZF{}, T0{}, g - 1, sw_a);
      fold(g, T1{}, sw_b);
    } else {
      fold(g - 1, T0{}, sw_a);
    }
  } else {
    for (int g = 0; g < KT; ++g) {
      step(g, T0{}, ZF{}, sw_a, NZ{}, T0{}, 0, sw_a);
      fold(g, T0{}, sw_a);
    }
  }

  // ---- epilogue
  if constexpr (kFullSteps) wait_vm<0>();  // trailing redundant reloads land before LDS is reused
  if constexpr (PART) {
    // partials of this K slice: 32 lanes of one accumulator row write 32
    // consecutive columns (128 bytes)
    int32_t* ws = acc_out + (int64_t)blockIdx.y * M * N;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = out_row(i, r), n = out_col(j);
          if (m < M && n < N) {
            if constexpr (GS == 0) ws[(int64_t)m * N + n] = acc[0][i][j][r];
            else ((float*)ws)[(int64_t)m * N + n] = facc[i][j][r];
          }
        }
    return;
  }
  if constexpr (ACC_OUT && GS == 0) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = out_row(i, r), n = out_col(j);
          if (m < M && n < N) acc_out[(int64_t)m * N + n] = INT4 ? (acc[0][i][j][r] >> 4) : acc[0][i][j][r];
        }
  }
  if (C == nullptr) return;
  if constexpr (OUT_DT != IC_DTYPE_F32) {
    // 16-bit outputs: finish each value in registers, stage the tile through
    // LDS row-major, then write whole rows with 16-byte stores.  s_a, bias and
    // the per-row weight scales are staged once per tile.  A 16-bit residual
    // is read into the same staging tile first, with 16-byte loads; each lane
    // then adds the residual of the slot it overwrites.
    bool staged = (((uintptr_t)C) & 15) == 0 && (ldc & 7) == 0 && (N & 7) == 0;
    bool res_lds = false;
    if constexpr (EPI) {
      res_lds = epi.res != nullptr;
      if (res_lds && (epi.res_dt == IC_DTYPE_F32 || (((uintptr_t)epi.res) & 15) != 0 || (epi.ldr & 7) != 0))
        staged = false;
    }
    if (staged) {
      constexpr int RS = TL::EPI_RS;
      constexpr int CPR = BN / 8;  // 16-byte chunks per tile row
      lds_barrier();  // every wave is done with the last stage
      u16* ot = (u16*)smem;
      float* sa_l = (float*)(smem + BM * RS * 2);
      float* b_l = sa_l + BM;
      float* sw_l = b_l + BN;
      float* rc_l = sw_l + BN;  // ROT: SmoothRot reciprocals of the tile's columns
      if (res_lds) {
        for (int c = tid; c < BM * CPR; c += kNT) {
          const int row = c / CPR, col = (c % CPR) * 8;
          const int m = m0 + row, n = n0 + col;
          if (m < M && n < N)
            *(v4u*)(ot + row * RS + col) = *(const v4u*)((const u16*)epi.res + (int64_t)m * epi.ldr + n);
        }
      }
      if (tid < BM) sa_l[tid] = pre_sa;
      if (tid < BN) {
        b_l[tid] = pre_b;
        if constexpr (GS == 0) sw_l[tid] = pre_sw;
        if constexpr (ROT != 0) rc_l[tid] = epi.sr_rcp != nullptr ? epi.sr_rcp[min(n0 + tid, N - 1)] : 1.0f;
      }
      __syncthreads();
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int nl = wc * WN + j * 32 + (lane & 31);
        const float b = b_l[nl];
        const float sw = GS == 0 ? sw_l[nl] : 0.0f;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int ml = wr * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            float v;
            if constexpr (GS == 0) {
              float a = (float)acc[0][i][j][r];
              if constexpr (INT4) a *= 0.0625f;
              v = a * (sa_l[ml] * sw);
            } else {
              v = facc[i][j][r] * sa_l[ml];
            }
            if (bias != nullptr) v = v + b;
            if constexpr (EPI) {
              v = epi_act(v, epi.act);
              if (res_lds) {
                const u16 r = ot[ml * RS + nl];
                v = v + (epi.res_dt == IC_DTYPE_F16 ? f16_to_f32(r) : bf16_to_f32(r));
              }
            }
            u16 h;
            if constexpr (OUT_DT == IC_DTYPE_F16) h = f32_to_f16(v);
            else h = f32_to_bf16(v);
            ot[ml * RS + nl] = h;
          }
          // with the epilogue options, keep the residual loads and activation
          // code of one 32x32 tile from being hoisted over all tiles
          if constexpr (EPI) __builtin_amdgcn_sched_barrier(0);
        }
      }
      __syncthreads();
      if constexpr (ROT != 0) {
        chain_rotate(ot, rc_l, (double*)(smem + TL::chain_xoff()));
        __syncthreads();
      }
#pragma unroll 4
      for (int c = tid; c < BM * CPR; c += kNT) {
        const int row = c / CPR, col = (c % CPR) * 8;
        const int m = m0 + row, n = n0 + col;
        if (m < M && n < N) *(v4u*)((u16*)C + (int64_t)m * ldc + n) = *(const v4u*)(ot + row * RS + col);
      }
      return;
    }
  }
  // Each lane stores 16 rows of one column per 32x32 tile; row offsets within
  // a tile stay in 32-bit arithmetic (the host bounds ldc).
  constexpr int ESZ = OUT_DT == IC_DTYPE_F32 ? 4 : 2;
  const bool full = m0 + BM <= M && n0 + BN <= N;
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int n = out_col(j);
    const int nc = min(n, N - 1);
    const float b = bias != nullptr ? ld_any_f32(bias, bias_dt, nc) : 0.0f;
    const float sw = GS == 0 ? s_w[nc] : 0.0f;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int mr0 = m0 + wr * WM + i * 32 + 4 * (lane >> 5);
      char* cb = (char*)C + ((int64_t)mr0 * ldc + n) * ESZ;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int dr = 8 * (r >> 2) + (r & 3);
        const int m = mr0 + dr;
        if (!full && (m >= M || n >= N)) continue;
        float v;
        if constexpr (GS == 0) {
          float a = (float)acc[0][i][j][r];
          if constexpr (INT4) a *= 0.0625f;
          v = a * (s_a[m] * sw);
        } else {
          v = facc[i][j][r] * s_a[m];
        }
        if (bias != nullptr) v = v + b;
        if constexpr (EPI) v = epi_apply(v, epi, m, n);
        st_from_f32<OUT_DT>(cb + dr * (int)ldc * ESZ, 0, v);
      }
      // keep the scale loads of one 32x32 tile from being hoisted over all tiles
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// Shape-generic fallback (any K, any alignment): one thread per output, exact
// int32 accumulation; same epilogue arithmetic as the MFMA kernel.  kil: the
// packed INT4 rows are in the K-interleaved nibble order.
template <bool INT4, int OUT_DT>
__global__ __launch_bounds__(256) void gemm_i8_generic_kernel(
    const int8_t* __restrict__ A, int64_t lda, const uint8_t* __restrict__ B, int64_t ldb,
    const float* __restrict__ s_a, const float* __restrict__ s_w, int G, int gsize,
    const void* __restrict__ bias, int bias_dt, void* __restrict__ C, int64_t ldc, int M, int N,
    int K, int32_t* __restrict__ acc_out, ic_epi epi, bool kil) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  const int m = blockIdx.y;
  if (n >= N || m >= M) return;
  const int8_t* a = A + (int64_t)m * lda;
  const uint8_t* b = B + (int64_t)n * ldb;
  // grouped scales fold once per block of gcd(group, 128) columns, as the
  // MFMA kernels do (once per 128-column stage, or per 64-K step)
  int fb = gsize, r128 = 128;
  while (r128 != 0) { const int t = fb % r128; fb = r128; r128 = t; }
  float facc = 0.0f;
  int acc = 0, acc_g = 0;
  for (int k = 0; k < K; ++k) {
    int w;
    if constexpr (INT4) {
      const int t = w4_nibble_index(k, kil);
      const int nib = (b[t >> 1] >> (4 * (t & 1))) & 0xf;
      w = nib >= 8 ? nib - 16 : nib;
    } else {
      w = (int8_t)b[k];
    }
    const int p = (int)a[k] * w;
    acc += p;
    if (G > 1) {
      acc_g += p;
      const int g = k / gsize;
      if ((k + 1) % fb == 0 || k + 1 == K) {
        facc = __builtin_fmaf((float)acc, s_w[(int64_t)n * G + g], facc);
        acc = 0;
      }
      if ((k + 1) % gsize == 0 || k + 1 == K) {
        if (acc_out) acc_out[((int64_t)g * M + m) * N + n] = acc_g;
        acc_g = 0;
      }
    }
  }
  if (G <= 1 && acc_out) acc_out[(int64_t)m * N + n] = acc;
  if (C == nullptr) return;
  float v = G > 1 ? facc * s_a[m] : (float)acc * (s_a[m] * s_w[n]);
  if (bias != nullptr) v = v + ld_any_f32(bias, bias_dt, n);
  v = epi_apply(v, epi, m, n);
  st_from_f32<OUT_DT>(C, (int64_t)m * ldc + n, v);
}

// Sum of the K-slice partials in slice order, then the operations of the
// unsplit epilogue; per-row-scale outputs are therefore bit-identical to an
// unsplit launch (exact int32 sums), grouped ones differ only in the order of
// the fp32 group-fold additions.
template <bool INT4, int GS, int OUT_DT>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(
    const int32_t* __restrict__ ws, int S, const float* __restrict__ s_a, const float* __restrict__ s_w,
    const void* __restrict__ bias, int bias_dt, void* __restrict__ C, int64_t ldc, int M, int N, ic_epi epi) {
  const int64_t MN = (int64_t)M * N;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= MN) return;
  const int m = (int)(i / N), n = (int)(i - (int64_t)m * N);
  float v;
  if constexpr (GS == 0) {
    int t = 0;
    for (int s = 0; s < S; ++s) t += ws[s * MN + i];
    float a = (float)t;
    if constexpr (INT4) a *= 0.0625f;
    v = a * (s_a[m] * s_w[n]);
  } else {
    const float* f = (const float*)ws;
    float t = f[i];
    for (int s = 1; s < S; ++s) t = t + f[s * MN + i];
    v = t * s_a[m];
  }
  if (bias != nullptr) v = v + ld_any_f32(bias, bias_dt, n);
  v = epi_apply(v, epi, m, n);
  st_from_f32<OUT_DT>(C, (int64_t)m * ldc + n, v);
}


// Workgroup rounds of a BM x BN tiling on the device's CUs times the tile
// area, times the tile's relative cost per output (percent): proportional to
// the run time of an MFMA-bound launch.
int64_t tiling_cost(const GemmArgs& g, int bm, int bn, int pct = 100) {
  const int64_t tiles = (int64_t)((g.M + bm - 1) / bm) * ((g.N + bn - 1) / bn);
  const int64_t cus = ic_num_cus();
  return (tiles + cus - 1) / cus * bm * bn * pct;
}

// Tile choice by tile-area rounds (tiling_cost).  Per-row W8A8 takes
// 256 x 192 where that fills the CUs in fewer rounds than 256 x 256
// (4096 x 3072: 256 tiles instead of 192 on 256 CUs).  INT4 / grouped:
// 256 x 128 (per-row INT4 also 256 x 256) unless 128 x 128 is cheaper; a 128 x 128 tile costs 1.44x more
// per output (measured on the Flux shapes), so it wins only when it fills CUs
// that 256 x 128 leaves idle (512 x 3072: 48 tiles of 256 x 128, 96 of
// 128 x 128 on 256 CUs).
struct TileShape { int bm, bn; };
TileShape tile_choice(const GemmArgs& g, bool grouped) {
  if (!g.int4 && !grouped) {
    if (g.M > 128 && g.N > 128)
      return tiling_cost(g, 256, 192) < tiling_cost(g, 256, 256) ? TileShape{256, 192} : TileShape{256, 256};
    return {128, 128};
  }
  if (g.M > 128 && tiling_cost(g, 256, 128) <= tiling_cost(g, 128, 128, 144)) {
    // per-row INT4 (no fold, int32 accumulators only) also fits 256 x 256,
    // ~0.9 of 256 x 128's cost per output (4608 x 3072: one round of 216
    // tiles, 195-200 us, against two of 432, 212 us)
    if (!grouped && g.N > 128 && tiling_cost(g, 256, 256, 90) < tiling_cost(g, 256, 128)) return {256, 256};
    return {256, 128};
  }
  return {128, 128};
}

// K slices for `tiles` workgroups over KT stages: minimise rounds of
// workgroups times stages per slice plus the partials' round trip through
// HBM (8 bytes per output and slice; ~3.6 MB per stage time) and, for grouped
// scales, the second kernel that adds the slices (~6 stage times: at M = 512,
// N = 3072, K = 3072 the unsplit grouped W4A8 took 24.3 us on packed and 19.4
// us on unpacked weights against 26.2 / 23.3 us split in two, and unsplit its
// outputs are the single fold chain's).  Only when the unsplit launch would
// leave more than half the CUs idle; 1 = no split.
int choose_splits(int64_t tiles, int KT, int64_t M, int64_t N, bool grouped) {
  const int64_t cus = ic_num_cus();
  if (tiles * 2 > cus || KT < 8) return 1;
  double best = (double)((tiles + cus - 1) / cus) * KT;
  int bs = 1;
  for (int S = 2; S <= 16 && KT / S >= 4; ++S) {
    const double c = (double)((tiles * S + cus - 1) / cus) * ((KT + S - 1) / S) + (double)S * M * N * 8.0 / 3.6e6 +
                     (grouped ? 6.0 : 0.0);
    if (c < best) { best = c; bs = S; }
  }
  return bs;
}

int splitk_plan(const GemmArgs& g, bool grouped) {
  const TileShape t = tile_choice(g, grouped);
  const int64_t tiles = (int64_t)((g.M + t.bm - 1) / t.bm) * ((g.N + t.bn - 1) / t.bn);
  return choose_splits(tiles, g.K / kBK, g.M, g.N, grouped);
}

template <class TL, int OUT_DT, bool ACC, bool PART, bool EPI>
hipError_t launch_kernel(const GemmArgs& g, int S, hipStream_t st) {
  const int tiles = ((g.M + TL::BM - 1) / TL::BM) * ((g.N + TL::BN - 1) / TL::BN);
  const size_t shm = TL::lds_bytes();
  static_assert(TL::lds_bytes() <= 160 * 1024, "LDS budget");
  auto kern = gemm_i8_kernel<TL, OUT_DT, ACC, PART, EPI>;
  static unsigned char lds_set[64];  // per device
  if (hipError_t e = ic_set_lds_limit((const void*)kern, (int)shm, lds_set)) return e;
  kern<<<dim3(tiles, S), dim3(kNT), shm, st>>>(g.A, g.lda, g.B, g.ldb, g.s_a, g.s_w, g.G, g.bias, g.bias_dt,
                                               g.C, g.ldc, g.M, g.N, g.K, PART ? (int32_t*)g.ws : g.acc_out, g.epi,
                                               g.kil ? kW4Kil : kW4Plain);
  return hipGetLastError();
}

template <class TL, int OUT_DT, bool ACC, bool EPI>
hipError_t launch_mfma(const GemmArgs& g, hipStream_t st) {
  if constexpr (!ACC) {
    const int S = g.ws != nullptr ? splitk_plan(g, TL::GS != 0) : 1;
    if (S > 1 && g.C != nullptr && g.ws_bytes >= (int64_t)S * g.M * g.N * 4) {
      hipError_t e = launch_kernel<TL, OUT_DT, false, true, EPI>(g, S, st);
      if (e != hipSuccess) return e;
      const int64_t MN = (int64_t)g.M * g.N;
      splitk_reduce_kernel<TL::INT4, TL::GS, OUT_DT><<<dim3((unsigned)((MN + 255) / 256)), dim3(256), 0, st>>>(
          (const int32_t*)g.ws, S, g.s_a, g.s_w, g.bias, g.bias_dt, g.C, g.ldc, g.M, g.N, g.epi);
      return hipGetLastError();
    }
  }
  return launch_kernel<TL, OUT_DT, ACC, false, EPI>(g, 1, st);
}

// Staged 16-bit output path of gemm_i8_big_kernel: output (and residual)
// 16-byte aligned, row strides and N multiples of 8.
bool big_out_ok(const GemmArgs& g) {
  if (g.out_dt == IC_DTYPE_F32 || (((uintptr_t)g.C) & 15) != 0 || (g.ldc & 7) != 0 || (g.N & 7) != 0) return false;
  return g.epi.res == nullptr ||
         (g.epi.res_dt != IC_DTYPE_F32 && (((uintptr_t)g.epi.res) & 15) == 0 && (g.epi.ldr & 7) == 0);
}

// Grouped INT4 on 288 x 192 tiles (gemm_i8_big_kernel) where their rounds of
// workgroups cost less than 256 x 128's: 4608 x 3072 (the Flux MLP-down and
// attention-projection shapes) fills the 256 CUs in one round of 256 tiles
// instead of two of 432.  That kernel writes 16-bit outputs through its LDS
// staging tile only, so the output (and a residual) must be 16-byte aligned
// with row strides and N multiples of 8.
// Its row counts: 256, 288 or 320 (8, 9 or 10 blocks of 16 rows per wave),
// whichever takes the fewest rounds x area, weighted per output against the
// 288-row tile by the operand bytes each reads (256 rows 1.05, 320 rows 0.99:
// at Wan's M = 32760 the per-row W8A8 288- and 320-row tiles took ~5 % less
// time per output than the 256-row one).  4096 rows: 16 tiles of 256; 4608:
// 16 of 288; Wan's 32760 x 5120: 103 x 27 tiles of 320, 11 rounds, against
// 114 x 27 of 288, 13 rounds.
struct BigPick { int tmb; int64_t cost; };
BigPick big_pick(const GemmArgs& g) {
  BigPick best{9, tiling_cost(g, 288, big::BN)};
  const int rows[2] = {8, 10}, pct[2] = {105, 99};
  for (int i = 0; i < 2; ++i) {
    const int64_t c = tiling_cost(g, 32 * rows[i], big::BN, pct[i]);
    if (c < best.cost) best = {rows[i], c};
  }
  return best;
}
int big_rows(const GemmArgs& g) { return big_pick(g).tmb; }
bool big_tile_ok(const GemmArgs& g) {
  if (g.M <= 128 || !big_out_ok(g)) return false;
  // per output the 288 x 192 tile costs ~0.93 of 256 x 128 (Wan FFN-down,
  // 32760 x 5120 x 14336: 13 rounds of it took as long as 20 of 256 x 128)
  return big_pick(g).cost * 93 / 100 < tiling_cost(g, 256, 128);
}

// Per-row weights (W8A8, per-row INT4) on the big tile where its rounds cost
// less than those of the tile_choice shape.  Per output of the 288-row tile
// it runs at ~0.9 of the W8A8 256 x 192 / 256 x 256 tiles (C1 4096 x 3072:
// 39.4 against 42.3 us on the same 256 x 192 tiling; 4608 x 3072 x 12288:
// 146 against 173 us, one round of 288 x 192 against one of 256 x 256; Wan
// qkv 32760 x 15360 x 5120: 2.60 against 2.81 ms) and ~0.8 of the per-row
// INT4 256 x 128 tile (4608 x 3072 x 12288: 141-148 against 192-198 us for
// 256 x 256): no fold, and the per-wave INT4 expansion runs beside 54 MFMAs a
// stage.  Not where a K split is planned (few tiles).
bool big_row_ok(const GemmArgs& g) {
  if (g.M <= 128 || g.N <= 128 || !big_out_ok(g)) return false;
  if (g.ws != nullptr && splitk_plan(g, false) > 1) return false;
  const TileShape t = tile_choice(g, false);
  const int tpct = t.bm == 128 ? (g.int4 ? 144 : 100) : (g.int4 && t.bn == 256 ? 90 : 100);
  return big_pick(g).cost * (g.int4 ? 80 : 90) / 100 < tiling_cost(g, t.bm, t.bn, tpct);
}

template <int OUT_DT, bool EPI, int MODE, int TMB, bool KIL>
hipError_t launch_big_t(const GemmArgs& g, hipStream_t st) {
  using RT = big::Rows<TMB, MODE>;
  const int tiles = ((g.M + RT::BM - 1) / RT::BM) * ((g.N + big::BN - 1) / big::BN);
  auto kern = gemm_i8_big_kernel<OUT_DT, EPI, MODE, TMB, KIL>;
  constexpr size_t shm = RT::lds_bytes;
  static unsigned char lds_set[64];  // per device
  if (hipError_t e = ic_set_lds_limit((const void*)kern, (int)shm, lds_set)) return e;
  kern<<<dim3(tiles), dim3(kNT), shm, st>>>(g.A, g.lda, g.B, g.ldb, g.s_a, g.s_w, g.G, g.bias, g.bias_dt, g.C,
                                            g.ldc, g.M, g.N, g.K, g.epi);
  return hipGetLastError();
}
template <int OUT_DT, bool EPI, int MODE, bool KIL = false>
hipError_t launch_big(const GemmArgs& g, hipStream_t st) {
  if constexpr (!KIL && MODE != big::ROW8 && MODE != big::G128I8) {
    if (g.kil) return ic_launch_big_kil(g, OUT_DT, EPI, MODE, st);
  }
  switch (big_rows(g)) {
    case 8: return launch_big_t<OUT_DT, EPI, MODE, 8, KIL>(g, st);
    case 10: return launch_big_t<OUT_DT, EPI, MODE, 10, KIL>(g, st);
    default: return launch_big_t<OUT_DT, EPI, MODE, 9, KIL>(g, st);
  }
}

template <bool INT4, int GS, int OUT_DT, bool ACC, bool EPI>
hipError_t pick_tile(const GemmArgs& g, hipStream_t st) {
  const TileShape t = tile_choice(g, GS != 0);
  if constexpr (GS != 0 && !ACC && OUT_DT != IC_DTYPE_F32) {
    // grouped packed INT4, or grouped int8 weights (INT4 unpacked to bytes)
    if (big_tile_ok(g)) return launch_big<OUT_DT, EPI, INT4 ? big::G128 : big::G128I8>(g, st);
  }
  if constexpr (GS == 0 && !ACC && OUT_DT != IC_DTYPE_F32) {
    if (big_row_ok(g)) return launch_big<OUT_DT, EPI, INT4 ? big::ROW4 : big::ROW8>(g, st);
  }
  if constexpr (!INT4 && GS == 0) {
    if (t.bm == 256 && t.bn == 192) return launch_mfma<Tile<256, 192, 4, 2, false, 0>, OUT_DT, ACC, EPI>(g, st);
    if (t.bm == 256) return launch_mfma<Tile<256, 256, 2, 2, false, 0>, OUT_DT, ACC, EPI>(g, st);
    return launch_mfma<Tile<128, 128, 2, 4, false, 0>, OUT_DT, ACC, EPI>(g, st);
  } else {
    if constexpr (INT4 && GS == 0) {
      if (t.bm == 256 && t.bn == 256) return launch_mfma<Tile<256, 256, 2, 2, true, 0>, OUT_DT, ACC, EPI>(g, st);
    }
    if (t.bm == 256) return launch_mfma<Tile<256, 128, 4, 3, INT4, GS>, OUT_DT, ACC, EPI>(g, st);
    return launch_mfma<Tile<128, 128, 2, 4, INT4, GS>, OUT_DT, ACC, EPI>(g, st);
  }
}

template <bool INT4, int GS, bool ACC, bool EPI>
hipError_t pick_out(const GemmArgs& g, hipStream_t st) {
  switch (g.out_dt) {
    case IC_DTYPE_F16: return pick_tile<INT4, GS, IC_DTYPE_F16, ACC, EPI>(g, st);
    case IC_DTYPE_BF16: return pick_tile<INT4, GS, IC_DTYPE_BF16, ACC, EPI>(g, st);
    default: return pick_tile<INT4, GS, IC_DTYPE_F32, ACC, EPI>(g, st);
  }
}

template <bool INT4, int OUT_DT>
hipError_t launch_generic_t(const GemmArgs& g, int gsize, hipStream_t st) {
  dim3 grid((unsigned)((g.N + 255) / 256), (unsigned)g.M);
  gemm_i8_generic_kernel<INT4, OUT_DT><<<grid, dim3(256), 0, st>>>(
      g.A, g.lda, g.B, g.ldb, g.s_a, g.s_w, g.G, gsize, g.bias, g.bias_dt, g.C, g.ldc, g.M, g.N, g.K,
      g.acc_out, g.epi, g.kil);
  return hipGetLastError();
}
template <bool INT4>
hipError_t launch_generic(const GemmArgs& g, int gsize, hipStream_t st) {
  switch (g.out_dt) {
    case IC_DTYPE_F16: return launch_generic_t<INT4, IC_DTYPE_F16>(g, gsize, st);
    case IC_DTYPE_BF16: return launch_generic_t<INT4, IC_DTYPE_BF16>(g, gsize, st);
    default: return launch_generic_t<INT4, IC_DTYPE_F32>(g, gsize, st);
  }
}

// The tile kernels form each DMA row offset within a tile (up to 320 rows) in
// 32-bit arithmetic, and each scale offset as n * G * 4.
bool dma_strides_ok(const GemmArgs& g) {
  return 320 * g.lda < (1LL << 31) && 320 * g.ldb < (1LL << 31) && (int64_t)g.N * g.G * 4 < (1LL << 31);
}

// Grouped scales take the MFMA kernels for group sizes that are multiples of
// 128: the fold runs once per 128-column stage with that stage's group scale
// (for 256, 384, ... each group's two or more stages fold separately).  The
// debug accumulator output writes one slab per group and needs 128.
bool mfma_shape_ok(const GemmArgs& g, int gsize) {
  if (g.K % kBK != 0) return false;
  if (g.G > 1 && (gsize % kBK != 0 || (g.acc_out != nullptr && gsize != kBK))) return false;
  // 16-byte DMA / vector loads need aligned bases and strides; packed INT4
  // rows are read 8 or 16 bytes at a time
  if (((uintptr_t)g.A & 15) || ((uintptr_t)g.B & 15) || (g.lda & 15) || (g.ldb & 15)) return false;
  return dma_strides_ok(g);
}

// Packed INT4 with groups of 64 or an odd multiple of 64 columns (the
// 128-column stages of the other MFMA kernels would straddle groups): the
// 288 x 192 kernel in its 64-block mode, when its operand and output layouts
// hold.  The debug accumulator output is not written by it.
bool big64_ok(const GemmArgs& g, int gsize) {
  if (!g.int4 || g.G <= 1 || gsize % 128 != 64 || g.K % kBK != 0 || g.acc_out != nullptr) return false;
  if (((uintptr_t)g.A & 15) || ((uintptr_t)g.B & 15) || (g.lda & 15) || (g.ldb & 15)) return false;
  return dma_strides_ok(g) && big_out_ok(g);
}

// Packed INT4 with groups of 32 or an odd multiple of 32 columns: the same
// kernel in its 32-column mode (two half-masked MFMAs per 64-K step).
bool big32_ok(const GemmArgs& g, int gsize) {
  if (!g.int4 || g.G <= 1 || gsize % 64 != 32 || g.K % kBK != 0 || g.acc_out != nullptr) return false;
  if (((uintptr_t)g.A & 15) || ((uintptr_t)g.B & 15) || (g.lda & 15) || (g.ldb & 15)) return false;
  return dma_strides_ok(g) && big_out_ok(g);
}

// Chained MLP epilogue launches (gemm_i8_chain.hip): 128 x 256 tiles, whose
// 256 columns hold whole R-blocks for R <= 256 and whose staging tile and
// fp64 exchange slices fit the LDS together.  The caller has checked the
// shape, the alignment of the staged output path and R.
template <class TL, int OUT_DT, int ROT>
hipError_t launch_chain_t(const GemmArgs& g, hipStream_t st) {
  const int tiles = ((g.M + TL::BM - 1) / TL::BM) * ((g.N + TL::BN - 1) / TL::BN);
  constexpr size_t shm = TL::chain_lds_bytes();
  static_assert(shm <= 160 * 1024, "LDS budget");
  auto kern = gemm_i8_kernel<TL, OUT_DT, false, false, true, ROT>;
  static unsigned char lds_set[64];  // per device
  if (hipError_t e = ic_set_lds_limit((const void*)kern, (int)shm, lds_set)) return e;
  kern<<<dim3(tiles), dim3(kNT), shm, st>>>(g.A, g.lda, g.B, g.ldb, g.s_a, g.s_w, g.G, g.bias, g.bias_dt, g.C,
                                            g.ldc, g.M, g.N, g.K, nullptr, g.epi, kW4Plain);
  return hipGetLastError();
}
template <class TL, int OUT_DT>
hipError_t launch_chain_r(const GemmArgs& g, int log4r, hipStream_t st) {
  switch (log4r) {
    case 2: return launch_chain_t<TL, OUT_DT, 2>(g, st);
    case 3: return launch_chain_t<TL, OUT_DT, 3>(g, st);
    default: return launch_chain_t<TL, OUT_DT, 4>(g, st);
  }
}
template <class TL>
hipError_t launch_chain(const GemmArgs& g, int log4r, hipStream_t st) {
  if (g.out_dt == IC_DTYPE_F16) return launch_chain_r<TL, IC_DTYPE_F16>(g, log4r, st);
  return launch_chain_r<TL, IC_DTYPE_BF16>(g, log4r, st);
}

// EPI: the activation / residual epilogue is compiled in (gemm_i8_epi.hip
// instantiates that set; gemm_i8.hip the plain one).
template <bool EPI>
int run_gemm_t(GemmArgs g, hipStream_t st, const char* who, bool force_generic) {
  if (g.M < 0 || g.N <= 0 || g.K <= 0 || g.lda < g.K || g.ldc < g.N)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: bad shape M=%d N=%d K=%d lda=%lld ldc=%lld", who, g.M,
                        g.N, g.K, (long long)g.lda, (long long)g.ldc);
  if (g.int4 ? (g.ldb * 2 < g.K) : (g.ldb < g.K))
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: weight row stride %lld too small for K=%d", who,
                        (long long)g.ldb, g.K);
  if (g.ldc >= (1LL << 24))
    return ic_set_error(IC_ERR_UNSUPPORTED, "%s: output row stride %lld too large", who, (long long)g.ldc);
  if (g.G < 1) return ic_set_error(IC_ERR_INVALID_ARG, "%s: num_groups must be >= 1", who);
  if (g.G > 1 && (g.K % g.G != 0))
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: K=%d not divisible by num_groups=%d", who, g.K, g.G);
  if (g.out_dt != IC_DTYPE_F16 && g.out_dt != IC_DTYPE_BF16 && g.out_dt != IC_DTYPE_F32)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: out dtype must be f16/bf16/f32", who);
  if (g.bias && g.bias_dt != IC_DTYPE_F16 && g.bias_dt != IC_DTYPE_BF16 && g.bias_dt != IC_DTYPE_F32)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: bias dtype must be f16/bf16/f32", who);
  if (g.M == 0) return IC_OK;
  if (!g.A || !g.B || !g.s_a || !g.s_w || (!g.C && !g.acc_out))
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: null pointer argument", who);
  const int gsize = g.K / g.G;
  hipError_t e;
  if (!force_generic && big64_ok(g, gsize)) {
    // groups of 64 (or an odd multiple of 64) columns: the 288 x 192 kernel
    // folding each 64-K step, at any M
    if (g.out_dt == IC_DTYPE_F16) e = launch_big<IC_DTYPE_F16, EPI, big::G64>(g, st);
    else e = launch_big<IC_DTYPE_BF16, EPI, big::G64>(g, st);
  } else if (!force_generic && big32_ok(g, gsize)) {
    // groups of 32 (or an odd multiple of 32) columns: the same kernel folding
    // each 32-column half step
    if (g.out_dt == IC_DTYPE_F16) e = launch_big<IC_DTYPE_F16, EPI, big::G32>(g, st);
    else e = launch_big<IC_DTYPE_BF16, EPI, big::G32>(g, st);
  } else if (!force_generic && mfma_shape_ok(g, gsize)) {
    if constexpr (EPI) {
      // the epilogue options never come with the debug accumulator output
      if (g.int4) e = g.G > 1 ? pick_out<true, 128, false, true>(g, st) : pick_out<true, 0, false, true>(g, st);
      else e = g.G > 1 ? pick_out<false, 128, false, true>(g, st) : pick_out<false, 0, false, true>(g, st);
    } else {
      const bool acc = g.acc_out != nullptr;
      if (g.int4) {
        if (g.G > 1) e = acc ? pick_out<true, 128, true, false>(g, st) : pick_out<true, 128, false, false>(g, st);
        else e = acc ? pick_out<true, 0, true, false>(g, st) : pick_out<true, 0, false, false>(g, st);
      } else {
        if (g.G > 1) e = acc ? pick_out<false, 128, true, false>(g, st) : pick_out<false, 128, false, false>(g, st);
        else e = acc ? pick_out<false, 0, true, false>(g, st) : pick_out<false, 0, false, false>(g, st);
      }
    }
  } else {
    e = g.int4 ? launch_generic<true>(g, gsize, st) : launch_generic<false>(g, gsize, st);
  }
  if (e != hipSuccess) return ic_set_error(IC_ERR_LAUNCH, "%s: %s", who, hipGetErrorString(e));
  return IC_OK;
}

}  // namespace
