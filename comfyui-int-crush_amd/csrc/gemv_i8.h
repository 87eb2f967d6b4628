// W8A8 / W4A8 small-batch GEMV (M <= 16 tokens): the per-block MFMA step and
// the epilogue shared by the GEMV on INT8 codes (gemv.hip) and the
// single-launch prep + GEMV (gemv_prep.h), and the former's kernel body.
//
// A 16-column block of outputs is computed by the four waves of a 256-thread
// workgroup, which split K in blocks of 128: two v_mfma_i32_16x16x64_i8 per
// block (rows = tokens, padded to 16; columns = outputs).  INT4 weights are
// expanded in registers to 16*q (two masks and a byte permute per 8 nibbles),
// the factor 16 removed exactly at the end.  Block sums are exact int32;
// grouped scales are folded afterwards in group order, so every output equals
// the tiled GEMM's (same formula, same rounding steps):
//   G == 1: f32(sum) * (s_a[m] * s_w[n]) (+ bias)
//   G  > 1: (fma chain over g of f32(acc_g) * s_w[n,g]) * s_a[m] (+ bias)
//
// Every lane of a wave reads 16 packed bytes (32 values) of one weight row per
// block, so a wave-wide load covers 16 rows x 64 bytes.
#pragma once
#include "ic_common.h"

namespace gemv {

constexpr int kGT = 256;   // threads per workgroup (4 waves)
constexpr int kGBK = 128;  // K per block
// XL: the M x K activation codes (at most kXlBytes) are staged in LDS once
// per workgroup, after the first batch of weight loads is issued, and read per
// block when used: fewer VGPRs, more waves per SIMD, more weight bytes in
// flight.
constexpr int kXlBytes = 16384;
constexpr int kOutRuntime = -1;  // OUT_DT: output dtype passed at run time

// One K block of one wave: MFMAs on the lane's 32 activation codes (av0, av1:
// K 32c .. 32c+31 of the block, c = lane / 16) and its 32 weights (INT4: the
// 16 packed bytes pwu; INT8: pwu and w1u).  Grouped (GS = 128, 64 or 32, the
// fold block gcd(group, 128)): the sums of the block's 128 / GS parts, each
// from the lanes holding that part's K range (the other lanes' codes zeroed),
// go to sacc[(b * 128 / GS + part)][M][16].  Per row (GS = 0) they accumulate
// in tot.  col = lane % 16.  sel: the nibble order of the packed weights.
template <bool INT4, int GS>
IC_DEV void mma_block(int b, const v4i& av0, const v4i& av1, const v4u& pwu, const v4i& w1u, int M, int c, int col,
                      int32_t* sacc, v4i& tot, W4Sel sel = kW4Plain) {
  v4i b0v, b1v;
  if constexpr (INT4) {
    uint32_t w[8];
    unpack8_x16(pwu.x, w[0], w[1], sel);
    unpack8_x16(pwu.y, w[2], w[3], sel);
    unpack8_x16(pwu.z, w[4], w[5], sel);
    unpack8_x16(pwu.w, w[6], w[7], sel);
    b0v = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
    b1v = v4i{(int)w[4], (int)w[5], (int)w[6], (int)w[7]};
  } else {
    b0v = __builtin_bit_cast(v4i, pwu);
    b1v = w1u;
  }
  if constexpr (GS != 0) {
    constexpr int NQ = 128 / GS;  // fold blocks per K block
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const bool keep = NQ == 1 || (c * NQ) / 4 == q;
      const v4i a0 = keep ? av0 : v4i{0, 0, 0, 0}, a1 = keep ? av1 : v4i{0, 0, 0, 0};
      v4i s = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0v, v4i{0, 0, 0, 0}, 0, 0, 0);
      s = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1v, s, 0, 0, 0);
      // D layout: lane holds rows 4*(lane/16) + i of column lane%16
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * c + i;
        if (r < M) sacc[((b * NQ + q) * M + r) * 16 + col] = s[i];
      }
    }
  } else {
    tot = __builtin_amdgcn_mfma_i32_16x16x64_i8(av0, b0v, tot, 0, 0, 0);
    tot = __builtin_amdgcn_mfma_i32_16x16x64_i8(av1, b1v, tot, 0, 0, 0);
  }
}

// Per-row mode: a wave's totals to sacc[wave][M][16].
IC_DEV void store_wave_totals(const v4i& tot, int wave, int M, int c, int col, int32_t* sacc) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 4 * c + i;
    if (r < M) sacc[(wave * M + r) * 16 + col] = tot[i];
  }
}

// Output (m, n0 + nl) from the sums of its 16-column block in sacc (after a
// barrier): dequant, bias, activation / residual, rounding to the output type.
// Grouped: the fold blocks of GS columns in K order, each with the scale of
// its group (gsize columns).
template <bool INT4, int GS, int OUT_DT>
IC_DEV void gemv_output(int m, int nl, const int32_t* sacc, int KB, int M, int n0, int N, const float* s_a,
                        const float* __restrict__ s_w, int G, int gsize, const void* __restrict__ bias, int bias_dt,
                        void* __restrict__ C, int out_dt, int64_t ldc, const ic_epi& epi) {
  const int no = n0 + nl;
  if (no >= N) return;
  float v;
  if constexpr (GS != 0) {
    const float* sw = s_w + (int64_t)no * G;
    const int nf = KB * (128 / GS), bpg = gsize / GS;  // fold blocks; per group
    float facc = 0.0f;
    if (bpg == 1) {  // group = fold block: scale addresses affine in the loop
      for (int f = 0; f < nf; ++f) {
        float s = sw[f];
        if constexpr (INT4) s *= 0.0625f;  // block sums hold 16 * the true sum
        facc = __builtin_fmaf((float)sacc[(f * M + m) * 16 + nl], s, facc);
      }
    } else {
      for (int f = 0, g = 0, r = 0; f < nf; ++f) {
        float s = sw[g];
        if constexpr (INT4) s *= 0.0625f;
        facc = __builtin_fmaf((float)sacc[(f * M + m) * 16 + nl], s, facc);
        if (++r == bpg) {
          r = 0;
          ++g;
        }
      }
    }
    v = facc * s_a[m];
  } else {
    const int t = ((sacc[(0 * M + m) * 16 + nl] + sacc[(1 * M + m) * 16 + nl]) +
                   sacc[(2 * M + m) * 16 + nl]) + sacc[(3 * M + m) * 16 + nl];
    float a = (float)t;
    if constexpr (INT4) a *= 0.0625f;
    v = a * (s_a[m] * s_w[no]);
  }
  if (bias != nullptr) v = v + ld_any_f32(bias, bias_dt, no);
  v = epi_apply(v, epi, m, no);
  if constexpr (OUT_DT == kOutRuntime) {
    if (out_dt == IC_DTYPE_F16) st_from_f32<IC_DTYPE_F16>(C, (int64_t)m * ldc + no, v);
    else if (out_dt == IC_DTYPE_BF16) st_from_f32<IC_DTYPE_BF16>(C, (int64_t)m * ldc + no, v);
    else st_from_f32<IC_DTYPE_F32>(C, (int64_t)m * ldc + no, v);
  } else {
    st_from_f32<OUT_DT>(C, (int64_t)m * ldc + no, v);
  }
}

// The GEMV on INT8 codes A [M, K] (row stride lda), one 16-column block per
// workgroup.  sacc: grouped: fold-block sums [K/GS][M][16]; per row: per-wave
// totals [4][M][16].  XL: xs receives the codes, copied after the first batch
// of weight loads is issued.
template <bool INT4, int GS, int OUT_DT, bool XL>
IC_DEV void gemv_i8_body(const int8_t* __restrict__ A, int64_t lda, const uint8_t* __restrict__ B, int64_t ldb,
                         const float* __restrict__ s_a, const float* __restrict__ s_w, int G, int gsize,
                         const void* __restrict__ bias, int bias_dt, void* __restrict__ C, int64_t ldc, int M, int N,
                         int K, const ic_epi& epi, int32_t* sacc, int8_t* xs, W4Sel sel) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n0 = blockIdx.x * 16;
  const int c = lane >> 4, col = lane & 15;
  const int n = min(n0 + col, N - 1);
  const int am = min(col, M - 1);  // token row fed by this lane (rows >= M repeat the last one)
  const int KB = K / kGBK;
  const int8_t* arow = XL ? xs + (int64_t)am * K + 32 * c : A + (int64_t)am * lda + 32 * c;
  const uint8_t* brow = B + (int64_t)n * ldb + (INT4 ? 16 * c : 32 * c);

  // Loads of up to kBatch blocks are issued before any of them is used, so a
  // wave keeps kBatch weight loads (plus activation loads) in flight.
  constexpr int kBatch = 8;
  v4i tot = {0, 0, 0, 0};
  if constexpr (XL) {
    v4u pw[kBatch];
    v4i w1[INT4 ? 1 : kBatch];
    auto load_batch = [&](int b0) {
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int b = b0 + 4 * u;
        if (b < KB) {  // uniform across the wave
          if constexpr (INT4) {
            pw[u] = *(const v4u*)(brow + (kGBK / 2) * b);
          } else {
            pw[u] = *(const v4u*)(brow + kGBK * b);
            w1[u] = *(const v4i*)(brow + kGBK * b + 16);
          }
        }
      }
    };
    // the first batch of weight loads is in flight while the codes are staged
    load_batch(wave);
    const int per_row = K / 16;  // 16-byte chunks
    for (int i = tid; i < M * per_row; i += kGT) {
      const int r = i / per_row, k16 = i - r * per_row;
      *(v4i*)(xs + (int64_t)r * K + 16 * k16) = *(const v4i*)(A + (int64_t)r * lda + 16 * k16);
    }
    __syncthreads();
    for (int b0 = wave; b0 < KB; b0 += 4 * kBatch) {
      if (b0 != wave) load_batch(b0);
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int b = b0 + 4 * u;
        if (b >= KB) break;
        mma_block<INT4, GS>(b, *(const v4i*)(arow + kGBK * b), *(const v4i*)(arow + kGBK * b + 16), pw[u],
                            w1[INT4 ? 0 : u], M, c, col, sacc, tot, sel);
      }
    }
  } else {
    for (int b0 = wave; b0 < KB; b0 += 4 * kBatch) {
      v4u pw[kBatch];
      v4i a0[kBatch], a1[kBatch], w1[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int b = b0 + 4 * u;
        if (b < KB) {  // uniform across the wave
          a0[u] = *(const v4i*)(arow + kGBK * b);
          a1[u] = *(const v4i*)(arow + kGBK * b + 16);
          if constexpr (INT4) {
            pw[u] = *(const v4u*)(brow + (kGBK / 2) * b);
          } else {
            pw[u] = *(const v4u*)(brow + kGBK * b);
            w1[u] = *(const v4i*)(brow + kGBK * b + 16);
          }
        }
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int b = b0 + 4 * u;
        if (b >= KB) break;
        mma_block<INT4, GS>(b, a0[u], a1[u], pw[u], w1[u], M, c, col, sacc, tot, sel);
      }
    }
  }
  if constexpr (GS == 0) store_wave_totals(tot, wave, M, c, col, sacc);
  __syncthreads();
  if (tid < 16 * M)
    gemv_output<INT4, GS, OUT_DT>(tid >> 4, tid & 15, sacc, KB, M, n0, N, s_a, s_w, G, gsize, bias, bias_dt, C,
                                  OUT_DT, ldc, epi);
}

}  // namespace gemv
