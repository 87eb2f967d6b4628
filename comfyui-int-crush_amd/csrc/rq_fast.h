// Fast path of the fused prep + quantize (the general kernel and the
// arithmetic it shares with this one are described in rotate_quant.hip).
// Included by one translation unit per activation dtype and instantiation set
// (rq_fast_{f16,bf16}{,_plain,_both}.hip, and rq_norm_{f16,bf16}{,_both}.hip
// for the normalising variants) so the sets compile in parallel.
#pragma once
#include "rq_common.h"

namespace {
using namespace rq;

// ===================================================================== fast path
// 16-bit activations with K_in % 16 == 0, K_w % 16 == 0, 16-byte aligned rows,
// factor and perm arrays, quantized output, no old-SmoothQuant divide.  Same
// arithmetic as rotate_quant_kernel, arranged for throughput:
//   * persistent workgroups walk rows r = blockIdx.x, +gridDim.x, ...; the
//     SmoothRot reciprocals of a thread's input positions and the gather
//     offsets of its output positions are loaded once into registers;
//   * the next row's activations are loaded into registers as soon as the
//     current row's values of that tile have been consumed, so HBM latency
//     overlaps a whole row of work;
//   * every 16-element run is entirely inside or outside the row, so the
//     per-element work is branch-free; the divide takes the IEEE slow path
//     only for a run holding a lane outside the proven fast-path range;
//   * rotated values are rounded once and kept as 16-bit values in an LDS row
//     buffer, which the gather reads directly (perm pre-scaled to byte offsets).

template <int DT> IC_DEV void unpack8(v4u a, float* o) {
  const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[2 * i] = bits16_f32<DT>((u16)(w[i] & 0xffffu));
    o[2 * i + 1] = bits16_f32<DT>((u16)(w[i] >> 16));
  }
}

// quantize 16 values of the activation type (|v| <= row abs-max) with scale
// s and r = RN32(1/s), and pack the codes little-endian
IC_DEV v4u quant16(const float* v, float s, float r) {
  uint32_t w[4];
#pragma unroll
  for (int d = 0; d < 4; ++d)
    w[d] = pack4_lo_bytes(quant_code_mk(v[4 * d], s, r), quant_code_mk(v[4 * d + 1], s, r),
                          quant_code_mk(v[4 * d + 2], s, r), quant_code_mk(v[4 * d + 3], s, r));
  return v4u{w[0], w[1], w[2], w[3]};
}

// Three instantiation sets (VAR): kRqPlain (no SmoothRot factors, no perm),
// kRqBoth (both, known at compile time) and kRqGeneral (either one, read at
// run time).  The plain kernels drop the per-run divide, its range checks,
// the gather's per-element LDS addressing and their registers; the
// compile-time flags of kRqBoth remove the unused gather path and the
// run-time branches (~9 % at the Flux MLP down-projection).  Two workgroups
// per CU while the per-thread constants fit half the register file (K_w <=
// 12288, or any width for plain rows); wider rows with factors or a perm keep
// one.
// Workgroup sums of two fp64 values (TH/64 waves; red holds 2 * TH/64
// doubles).  The caller guarantees red is no longer being read (a barrier at
// the top of the row, or a copy of red per row parity), so one barrier
// suffices.
template <int TH>
IC_DEV void block_sum2_f64(double& a, double& b, double* red) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    a += __shfl_xor(a, o, 64);
    b += __shfl_xor(b, o, 64);
  }
  if ((threadIdx.x & 63) == 0) {
    red[2 * (threadIdx.x >> 6)] = a;
    red[2 * (threadIdx.x >> 6) + 1] = b;
  }
  __syncthreads();
  a = red[0];
  b = red[1];
#pragma unroll
  for (int w = 1; w < TH / 64; ++w) {
    a += red[2 * w];
    b += red[2 * w + 1];
  }
}

// TH threads per workgroup (256; 192 = three waves for rows of up to 3072 or
// 6144 values, 320 = five waves for rows of 4097..5120 values and 448 = seven
// for 12289..14336, all with R <= 1024, whose Hadamard exchange stays inside a
// wave): a tile is TH * 16 positions.  For R = 1024 a wave's 64 x 16 positions are exactly one block,
// so its last digit is exchanged through the wave's own slice of the LDS
// buffer, without a workgroup barrier.
//
// NORM (IC_NORM_LAYER / IC_NORM_RMS, ic_norm_rotate_quantize): before the
// prep, the row is normalised and rounded once to DT,
//   y = RN_dt(f32(f32(f32(x - mean) * rstd) * nw[k]) + nb[k])     (LayerNorm)
//   y = RN_dt(f32(f32(x * rstd) * nw[k]) + nb[k])                  (RMSNorm)
// (nw / nb optional), mean = RN32(S1 / K_in) and rstd = RN32(1 / sqrt(V / K_in
// + eps)) from fp64 sums over the row the registers already hold: one pass,
// V = S2 - S1^2 / K_in with S1 = sum x, S2 = sum x^2 (the sums of 16-bit
// values are exact in fp64 for any realistic row).  The prep
// then treats y as its input: the same arithmetic as the chain normalise ->
// activation tensor -> rotate_quantize, without the tensor.
// (the 768-thread workgroup, and the two-tile 448 / 512-thread ones with a
// row buffer, leave LDS for one workgroup per CU, which their launch bounds
// say)
template <int DT, int LOG4R, int NT, int VAR, int TH>
constexpr int rq_fast_min_wgs() {
  const bool wave_local = VAR == kRqPlain && LOG4R >= 3 && LOG4R <= 5 && NT <= 2;
  if (TH >= 768 || (TH >= 448 && NT >= 2 && !wave_local)) return 1;
  return (NT <= 3 || VAR == kRqPlain) ? 2 : 1;
}
template <int DT, int LOG4R, int NT, int VAR, int TH, int NORM = 0>
__global__ __launch_bounds__(TH, (rq_fast_min_wgs<DT, LOG4R, NT, VAR, TH>())) void rq_fast_kernel(
    const u16* __restrict__ x, int64_t ldx, int M, int K_in, int K_r,
    const float* __restrict__ sr_rcp, const float* __restrict__ sr_f, int K_w,
    const int32_t* __restrict__ perm, int8_t* __restrict__ q_out, int64_t ldq,
    float* __restrict__ s_out, const float* __restrict__ nw, const float* __restrict__ nb, float eps) {
  constexpr int RC = LOG4R <= 2 ? 0 : (LOG4R <= 4 ? 1 : (LOG4R == 5 ? 3 : 2));
  constexpr bool XCH = LOG4R >= 3;
  constexpr int kTile = TH * 16;  // positions per tile
  static_assert(TH == 256 || (TH % 64 == 0 && LOG4R <= 5), "cross-wave rotation needs four waves");
  // WLR: rows without a perm whose rotation stays inside each wave's 1024
  // positions (R = 64..1024 with the DMA-staged slices, at most two tiles)
  // keep their rounded values in the upper half of the wave's own exchange
  // slice instead of a row buffer: the quantization then reads only what
  // its own wave wrote, and the workgroup needs no row-sized buffer (the
  // Wan FFN-down rows fit two workgroups per CU instead of one).
  constexpr bool WLR = VAR == kRqPlain && XCH && LOG4R <= 5 && NT <= 2;
  // DBR: the row buffer and the reduction slots alternate between two copies
  // by row parity, so no barrier is needed at the top of a row: a wave that
  // writes row r + 2's copy has passed row r + 1's abs-max barrier, which no
  // wave reaches before it has finished reading row r's.  For rotations that
  // stay inside each wave (R <= 1024), where the second row buffer leaves the
  // workgroups the LDS admits per CU unchanged (WLR kernels have none).
  //
  // XROT (R = 64 / 256 with a row buffer): the exchange buffer without the
  // 16 doubles of padding per 256 positions (tslot), where that is what lets
  // the second row buffer fit and more than one workgroup shares a CU (one
  // 768-thread workgroup per CU measured slower with it).  The padding put
  // the four 16-lane groups of a wave 128 bytes apart modulo the 512 bytes of
  // the LDS banks for the transposed reads.  Without it the groups' blocks
  // lie 2304 bytes apart (256 mod 512), so groups 0 and 2 (and 1 and 3) would
  // meet; instead groups 2 and 3 of each wave read their 16 rows in the order
  // h ^ 8, a further 1152 bytes (128 mod 512) away: the four reads of a row
  // land at 0, 256, 128 and 384 mod 512.  Those lanes' registers then hold
  // rows h ^ 8: the radix-4 digit on bits 2-3 maps register a to logical
  // a ^ 2, and y_i = s/2 - x_(3-i) commutes with that relabeling
  // (3 - (a ^ 2) = (3 - a) ^ 2), so the butterflies run unchanged and only
  // the row-buffer stores (and the test of pad positions) use the logical
  // index j ^ 8.
  constexpr int kRowLen = WLR ? 8 : rowbuf_len<NT, kTile>();
  constexpr int kWgCap = 1024 / TH;  // ~16 waves per CU at these kernels' register counts
  // the reduction slots (NB copies) and 32 bytes of alignment
  constexpr int kSlots1 = (TH / 64) * 4 + (NORM != 0 ? 2 * (TH / 64) : 1) * 8 +
                          (DT == IC_DTYPE_BF16 && LOG4R == 6 ? 2 * (TH / 64) : 1) * 4 + 32;
  constexpr int kSlots2 = kSlots1 + (TH / 64) * 4 + (NORM != 0 ? 2 * (TH / 64) : 1) * 8;
  // workgroups per CU with one or two row buffers and an exchange buffer of
  // XB bytes (LDS is allocated in 512-byte granules)
  constexpr auto occ = [](int xb, int nbuf) {
    const int lds = (xb + 2 * nbuf * kRowLen + (nbuf == 1 ? kSlots1 : kSlots2) + 511) / 512 * 512;
    return 163840 / lds < kWgCap ? 163840 / lds : kWgCap;
  };
  constexpr auto dbr_fits = [occ](int xb) { return occ(xb, 2) >= 1 && occ(xb, 2) >= occ(xb, 1); };
  constexpr int kXbPad = XCH ? 8 * xbuf_doubles<kTile>() : 16;
  constexpr int kXbTight = XCH ? 8 * tslot_doubles<kTile>() : 16;
  constexpr bool XROT = XCH && (LOG4R == 3 || LOG4R == 4) && !WLR && kWgCap >= 2 && !dbr_fits(kXbPad) &&
                        dbr_fits(kXbTight);
  constexpr bool DBR = LOG4R <= 5 && (WLR || dbr_fits(XROT ? kXbTight : kXbPad));
  __shared__ double xbuf[XCH ? (XROT ? tslot_doubles<kTile>() : xbuf_doubles<kTile>()) : 2];
  auto xs = [](int p) { return XROT ? tslot(p) : xslot(p); };
  constexpr int NB = DBR ? 2 : 1;
  __shared__ __attribute__((aligned(16))) u16 rowbuf_all[(DBR && !WLR) ? 2 : 1][kRowLen];
  __shared__ float red_all[NB][TH / 64];
  __shared__ double red_d_all[NB][NORM != 0 ? 2 * (TH / 64) : 1];
  __shared__ uint32_t xred[DT == IC_DTYPE_BF16 && LOG4R == 6 ? 2 * (TH / 64) : 1];

  constexpr bool PLAIN = VAR == kRqPlain;
  const int t = threadIdx.x;
  const bool has_sr = VAR == kRqBoth || (VAR == kRqGeneral && sr_rcp != nullptr);
  const bool has_perm = VAR == kRqBoth || (VAR == kRqGeneral && perm != nullptr);

  // ---- per-workgroup constants (not allocated by PLAIN kernels)
  constexpr int NTC = PLAIN ? 1 : NT;
  float rc[NTC][16];
  uint32_t po[NTC][8];
#pragma unroll
  for (int c = 0; c < NTC; ++c) {
    if constexpr (PLAIN) break;
    const int p0 = c * kTile + 16 * t;
#pragma unroll
    for (int j = 0; j < 16; ++j) rc[c][j] = 1.0f;
    if (has_sr && p0 < K_in) {
      const v4f* src = (const v4f*)(sr_rcp + p0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const v4f r = src[i];
        rc[c][4 * i] = r.x; rc[c][4 * i + 1] = r.y; rc[c][4 * i + 2] = r.z; rc[c][4 * i + 3] = r.w;
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) po[c][i] = 0;
    if (has_perm && p0 < K_w) {
      const v4u* src = (const v4u*)(perm + p0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const v4u r = src[i];
        const uint32_t e[4] = {r.x, r.y, r.z, r.w};
        uint32_t off[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) off[k] = 2u * (uint32_t)rbaddr(e[k] < (uint32_t)K_w ? (int)e[k] : 0);  // malformed -> position 0
        po[c][2 * i] = off[0] | (off[1] << 16);
        po[c][2 * i + 1] = off[2] | (off[3] << 16);
      }
    }
  }

  // Activation runs of the next row are fetched while the current row is
  // processed; runs past K_in (only in the last, partial tiles) are zero.
  //   kDma (R = 64..1024, whose exchanges stay inside each wave's own 1024-
  //   position slice of xbuf): global -> LDS DMA into that slice, issued once
  //   the row's last exchange has been read, waited for with an explicit
  //   vmcnt at the top of the next row and copied into registers there.  The
  //   compiler otherwise moved register prefetches into fresh registers in
  //   mid-row, which waited for the loads (and the previous row's stores) there.
  //   Otherwise: register loads one row ahead.
  constexpr bool kDma = XCH && LOG4R <= 5;
  v4u xr[NT][2];
  auto load_x = [&](int r, int c) {
    const int p0 = c * kTile + 16 * t;
    if (p0 < K_in) {
      const v4u* src = (const v4u*)(x + (int64_t)r * ldx + p0);
      xr[c][0] = src[0];
      xr[c][1] = src[1];
    } else {
      xr[c][0] = xr[c][1] = v4u{0, 0, 0, 0};
    }
  };
  // DMA staging: the NT tiles' 32 bytes per lane at slice + 2048 c + 16 lane
  // (first 8 values) and + 1024 (last 8); NT * 2 KB fit the 8 KB slice.
  const int wave_u = __builtin_amdgcn_readfirstlane(t >> 6);
  const int lane = t & 63;
  char* const slice = (char*)(xbuf + (XCH ? xs(1024 * wave_u) : 0));
  const uint32_t slice_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)slice;
  auto stage_row = [&](int r) {
    const u16* rb = x + (int64_t)r * ldx;
#pragma unroll
    for (int c = 0; c < NT; ++c) {
      if (c * kTile >= K_in) break;  // uniform
      // pad runs read the row's last 16 values (a valid address) and are zeroed after
      const uint32_t voff = 2u * (uint32_t)min(c * kTile + 16 * t, K_in - 16);
      dma16_lds(voff, rb, slice_lds + (uint32_t)(c * 2048));
      dma16_lds(voff + 16u, rb, slice_lds + (uint32_t)(c * 2048 + 1024));
    }
  };
  // WLR: byte offset in the slice of wave-local position q of tile c (tiles
  // of 1024 + 64 values from byte 4096; the slice holds 1216 doubles)
  auto wlr_off = [](int c, int q) { return 4096 + 2176 * c + 2 * (q + 16 * (q >> 8)); };
  static_assert(!WLR || 4096 + 2176 * NT <= 8 * 1216, "WLR rows fit the exchange slice");
  // Vector-memory operations each wave issues after its DMA of a row: one
  // 16-byte code store per tile that every lane of every wave stores (plus,
  // on some waves, pad-tile stores and the scale store, which only add).
  const int kStoresAfterDma = min(K_w / kTile, NT);
  if constexpr (!PLAIN) {
    if constexpr (kDma) {
      // the constants' loads complete here (the compiler waits for them
      // before these reads); an empty asm then is their last writer, so no
      // wait for them is carried into the row loop, where it would also
      // wait for the DMA and the previous row's stores
#pragma unroll
      for (int c = 0; c < NTC; ++c) {
#pragma unroll
        for (int j = 0; j < 16; ++j) asm volatile("" : "+v"(rc[c][j]));
#pragma unroll
        for (int i = 0; i < 8; ++i) asm volatile("" : "+v"(po[c][i]));
      }
    }
  }
  int row = blockIdx.x;
  if (row < M) {
    if constexpr (kDma) {
      stage_row(row);
    } else {
#pragma unroll
      for (int c = 0; c < NT; ++c)
        if (c * kTile < K_in) load_x(row, c);
    }
  }
  bool first_row = true;
  int parity = 0;

  for (; row < M; row += gridDim.x, parity ^= (DBR ? 1 : 0)) {
    const int next = row + gridDim.x;
    u16* const rowbuf = rowbuf_all[WLR ? 0 : parity];
    float* const red = red_all[parity];
    double* const red_d = red_d_all[parity];
    if constexpr (!DBR) __syncthreads();  // the previous row's gather is done with rowbuf and red
    // Wave priority ramps down over the row (3 after the barrier, 2 in the
    // rotation, 1 in the rounding, 0 from the row scale on).  The SIMDs
    // otherwise issue oldest-wave-first, so each SIMD's youngest wave finished
    // its rotation last, alone, while the others waited at the abs-max
    // barrier; a wave that is ahead now yields to the ones behind it
    // (measured 7-12 % faster at C3, outputs unchanged).
    __builtin_amdgcn_s_setprio(3);
    if constexpr (kDma) {
      // this row's activations: DMA issued during the previous row (or above),
      // followed since by at least kStoresAfterDma stores of this wave
      if (first_row) wait_vm_imm<0>();
      else wait_vm_n(kStoresAfterDma);
      first_row = false;
#pragma unroll
      for (int c = 0; c < NT; ++c) {
        if (c * kTile >= K_in) break;  // uniform
        if (c * kTile + 16 * t < K_in) {
          xr[c][0] = *(const v4u*)(slice + c * 2048 + lane * 16);
          xr[c][1] = *(const v4u*)(slice + c * 2048 + 1024 + lane * 16);
        } else {
          xr[c][0] = xr[c][1] = v4u{0, 0, 0, 0};
        }
      }
    }
    float n_mean = 0.0f, n_rstd = 1.0f;
    if constexpr (NORM != 0) {
      // row statistics from the registers (runs at or past K_in add nothing)
      double s1 = 0.0, s2 = 0.0;
#pragma unroll
      for (int c = 0; c < NT; ++c) {
        if (c * kTile + 16 * t >= K_in) continue;
        float xs[16];
        unpack8<DT>(xr[c][0], xs);
        unpack8<DT>(xr[c][1], xs + 8);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const double d = (double)xs[j];
          if constexpr (NORM == IC_NORM_LAYER) s1 += d;
          s2 += d * d;
        }
      }
      block_sum2_f64<TH>(s1, s2, red_d);
      if constexpr (NORM == IC_NORM_LAYER) {
        const double mean = s1 / K_in;
        const double var = __builtin_fmax(s2 / K_in - mean * mean, 0.0);
        n_mean = (float)mean;
        n_rstd = (float)(1.0 / __builtin_sqrt(var + (double)eps));
      } else {
        n_rstd = (float)(1.0 / __builtin_sqrt(s2 / K_in + (double)eps));
      }
    }
    float amax = 0.0f;
    uint32_t zs[WLR ? NT : 1][8];  // WLR: this lane's rounded values, packed as they are written
#pragma unroll
    for (int c = 0; c < NT; ++c) {
      const int base = c * kTile;
      if (base >= K_w) break;  // uniform
      const int p0 = base + 16 * t;
      double v[16];
      if (base < K_in) {  // uniform: the tile holds input values
        const v4u xa = xr[c][0], xb = xr[c][1];
        if (!kDma && next < M) load_x(next, c);
        float xs[16];
        unpack8<DT>(xa, xs);
        unpack8<DT>(xb, xs + 8);
        float xn[NORM != 0 ? 16 : 1];  // normalised run, the divide's input
        if constexpr (NORM != 0) {
          if (p0 < K_in) {  // pad runs stay zero
            float w[16], b[16];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const v4f wv = nw != nullptr ? ((const v4f*)(nw + p0))[i] : v4f{1.0f, 1.0f, 1.0f, 1.0f};
              const v4f bv = nb != nullptr ? ((const v4f*)(nb + p0))[i] : v4f{0.0f, 0.0f, 0.0f, 0.0f};
              w[4 * i] = wv.x; w[4 * i + 1] = wv.y; w[4 * i + 2] = wv.z; w[4 * i + 3] = wv.w;
              b[4 * i] = bv.x; b[4 * i + 1] = bv.y; b[4 * i + 2] = bv.z; b[4 * i + 3] = bv.w;
            }
#pragma unroll
            for (int j = 0; j < 16; ++j) {
              float y = NORM == IC_NORM_LAYER ? (xs[j] - n_mean) * n_rstd : xs[j] * n_rstd;
              if (nw != nullptr) y = y * w[j];
              if (nb != nullptr) y = y + b[j];
              xs[j] = round_to_dt<DT>(y);
            }
          }
#pragma unroll
          for (int j = 0; j < 16; ++j) xn[j] = xs[j];
        }
        // bf16: the run's |x| extremes for the flush rule, formed with the
        // divide's own range test where there is one
        Bf16RunStats fst{0u, 0.0f};
        bool fst_ok = false;
        if (has_sr) {
          // fast path valid for products p = RN32(x * rcp) in DT's normal
          // range, which |RN_dt(p)| > min normal guarantees (RN_dt moves p by
          // at most half a DT ulp); zeros, pad runs and non-finite values
          // take the exact path, which returns the same signed zero
          float hmin = __builtin_huge_valf();
          uint32_t hmax_bits = 0u;  // bf16: largest |x| as bits (NaN > inf > finite)
          if constexpr (DT == IC_DTYPE_BF16) {
            // pairs rounded by one packed conversion; the extremes of |x| as
            // packed 16-bit integers (bf16 bits without the sign order as the
            // values, NaN above inf; a NaN minimum sends the run to the exact
            // path, as the non-finite test would)
            typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
            u16x2 hmx = {0, 0}, hmn = {0xffff, 0xffff};
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              const uint32_t w = pack2_bits16<DT>(xs[2 * i] * rc[PLAIN ? 0 : c][2 * i],
                                                  xs[2 * i + 1] * rc[PLAIN ? 0 : c][2 * i + 1]);
              xs[2 * i] = __uint_as_float(w << 16);
              xs[2 * i + 1] = __uint_as_float(w & 0xffff0000u);
              const u16x2 a = __builtin_bit_cast(u16x2, w & 0x7fff7fffu);
              hmx = __builtin_elementwise_max(hmx, a);
              hmn = __builtin_elementwise_min(hmn, a);
            }
            hmax_bits = (uint32_t)(hmx.x > hmx.y ? hmx.x : hmx.y) << 16;
            hmin = __uint_as_float((uint32_t)(hmn.x < hmn.y ? hmn.x : hmn.y) << 16);
          } else {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
              xs[j] = round_to_dt<DT>(xs[j] * rc[PLAIN ? 0 : c][j]);
              hmin = __builtin_fminf(hmin, __builtin_fabsf(xs[j]));
            }
          }
          const bool nonfinite = DT == IC_DTYPE_BF16 && hmax_bits >= 0x7f800000u;
          fst = Bf16RunStats{hmax_bits, hmin};
          fst_ok = true;
          if (__builtin_expect(!(hmin > dt_min_normal<DT>()) || nonfinite, 0)) {
            fst_ok = false;  // the exact path below replaces the run
            if (p0 < K_in) {
              float xo[16];
              if constexpr (NORM != 0) {
#pragma unroll
                for (int j = 0; j < 16; ++j) xo[j] = xn[j];
              } else {
                unpack8<DT>(xa, xo);
                unpack8<DT>(xb, xo + 8);
              }
#pragma unroll
              for (int j = 0; j < 16; ++j) xs[j] = div_round_dt<DT>(xo[j], rc[PLAIN ? 0 : c][j], sr_f, p0 + j);
            } else {
#pragma unroll
              for (int j = 0; j < 16; ++j) xs[j] = 0.0f;
            }
          }
        }
        if constexpr (DT == IC_DTYPE_BF16 && LOG4R >= 2) {
          if (!fst_ok) fst = bf16_run_stats(xs);
          bf16_flush_small<LOG4R, TH>(xs, xred, fst);
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = (double)xs[j];
      } else {
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = 0.0;
      }
      if (c == 0) __builtin_amdgcn_s_setprio(2);
      // ---- block Hadamard (same digit layout as rotate_quant_kernel)
      if constexpr (LOG4R >= 2) { stage_lo(v); stage_hi(v); }
      if constexpr (XCH) {
        // digits 2-3: transpose among 16 lanes of one wave (no workgroup barrier)
#pragma unroll
        for (int j = 0; j < 16; ++j) xbuf[xs(16 * t + j)] = v[j];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const int g = t >> 4, l = t & 15;
        if constexpr (XROT) {
          // row h ^ 8 for groups 2 and 3 of the wave: tslot(256 g + 16 (h ^ 8) + l)
          const int gp = (g >> 1) & 1;
          const int r_lo = 288 * g + 144 * gp + l, r_hi = 288 * g - 144 * gp + l;
#pragma unroll
          for (int h = 0; h < 16; ++h) v[h] = xbuf[(h < 8 ? r_lo : r_hi) + 18 * h];
        } else {
#pragma unroll
          for (int h = 0; h < 16; ++h) v[h] = xbuf[xslot(256 * g + 16 * h + l)];
        }
        stage_lo(v);
        if constexpr (LOG4R >= 4) stage_hi(v);
        if constexpr (LOG4R == 5) {
          // digit 4 spans the wave's four 256-groups: element 4i+b of lane ln
          // takes position 1024w + 256b + 4ln + i (tile_pos<3>)
#pragma unroll
          for (int h = 0; h < 16; ++h) xbuf[xslot(256 * g + 16 * h + l)] = v[h];
          __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
          __builtin_amdgcn_wave_barrier();
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
          const int wb = 1024 * (t >> 6) + 4 * (t & 63);
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int b = 0; b < 4; ++b) v[4 * i + b] = xbuf[xslot(wb + 256 * b + i)];
          stage_lo(v);
          __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
          __builtin_amdgcn_wave_barrier();
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        } else if constexpr (LOG4R >= 6) {
          // digits 4-5 span all four waves
#pragma unroll
          for (int h = 0; h < 16; ++h) xbuf[xslot(256 * g + 16 * h + l)] = v[h];
          __syncthreads();
#pragma unroll
          for (int gg = 0; gg < 16; ++gg) v[gg] = xbuf[xslot(256 * gg + t)];
          stage_lo(v);
          stage_hi(v);
          __syncthreads();  // every wave has read xbuf before the next tile rewrites it
        } else {
          __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
          __builtin_amdgcn_wave_barrier();
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
      }
      if (c + 1 == NT || base + kTile >= K_w) __builtin_amdgcn_s_setprio(1);
      // ---- round once to DT: RN32 first; exact round-to-odd for the rare runs
      // holding a DT rounding boundary, a tiny value or a zero, and for the
      // runs of a tile that reaches into the pad to K_w (zeroed there)
      float z[16];
      float zmin = __builtin_huge_valf(), zmax = 0.0f;
      uint32_t bmin = 0xffffffffu;  // zero iff some z[j] is a DT boundary
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        z[j] = (float)v[j];
        zmin = __builtin_fminf(zmin, __builtin_fabsf(z[j]));
        zmax = __builtin_fmaxf(zmax, __builtin_fabsf(z[j]));
        const uint32_t key = rn32_boundary_key<DT>(z[j]);
        bmin = bmin < key ? bmin : key;
      }
      if (__builtin_expect(bmin == 0u || !(zmin >= dt_min_normal<DT>()) || base + kTile > K_r, 0)) {
        zmax = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          z[j] = rto24(v[j]);
          const int jl = XROT ? (j ^ (8 * ((t >> 5) & 1))) : j;  // logical index of register j
          if (base + kTile > K_r && base + tile_pos<(LOG4R == 0 ? 0 : RC)>(t, jl) >= K_r) z[j] = 0.0f;
          zmax = __builtin_fmaxf(zmax, __builtin_fabsf(z[j]));
        }
      }
      amax = __builtin_fmaxf(amax, zmax);
      if constexpr (WLR) {
        // kept until every exchange of the row is done (the next tile's
        // exchange reuses the whole slice); pairs in the store order below
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          if constexpr (RC == 3) zs[c][i] = pack2_bits16<DT>(z[(i & 1) * 8 + (i >> 1)], z[(i & 1) * 8 + (i >> 1) + 4]);
          else zs[c][i] = pack2_bits16<DT>(z[2 * i], z[2 * i + 1]);
        }
      } else if constexpr (LOG4R == 0 || RC == 0) {
        // 16 contiguous positions per thread: two 16-byte stores
        uint32_t w[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = pack2_bits16<DT>(z[2 * i], z[2 * i + 1]);
        v4u* dst = (v4u*)(rowbuf + rbaddr(base + 16 * t));
        dst[0] = v4u{w[0], w[1], w[2], w[3]};
        dst[1] = v4u{w[4], w[5], w[6], w[7]};
      } else if constexpr (RC == 3) {
        // elements b, 4+b, 8+b, 12+b are four consecutive positions: one 8-byte store
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const uint32_t lo = pack2_bits16<DT>(z[b], z[4 + b]);
          const uint32_t hi = pack2_bits16<DT>(z[8 + b], z[12 + b]);
          *(v2u*)(rowbuf + rbaddr(base + tile_pos<3>(t, b))) = v2u{lo, hi};
        }
      } else if constexpr (XROT) {
        // registers 2i, 2i + 1 hold logical elements (2i) ^ 8g', (2i + 1) ^ 8g'
        // (g' = 1 in groups 2 and 3 of the wave), i.e. 128 positions further
        // (i < 4) or back (i >= 4) there; all inside the lane's 256-position block
        static_assert(RC == 1, "XROT stores");
        const int gp = (t >> 5) & 1;
        u16* const rl = rowbuf + rbaddr(base + tile_pos<1>(t, 0)) + 128 * gp;
        u16* const rh = rowbuf + rbaddr(base + tile_pos<1>(t, 0)) - 128 * gp;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t w = pack2_bits16<DT>(z[2 * i], z[2 * i + 1]);
          u16* const r = i < 4 ? rl : rh;
          r[32 * i] = (u16)w;
          r[32 * i + 16] = (u16)(w >> 16);
        }
      } else {
        // pairs rounded by one packed conversion, stored as two 16-bit halves
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t w = pack2_bits16<DT>(z[2 * i], z[2 * i + 1]);
          rowbuf[rbaddr(base + tile_pos<RC>(t, 2 * i))] = (u16)w;
          rowbuf[rbaddr(base + tile_pos<RC>(t, 2 * i + 1))] = (u16)(w >> 16);
        }
      }
    }

    if constexpr (WLR) {
      // into the slice's upper part (the next row's DMA fills bytes 0..4095):
      // wave-local position q of tile c at byte wlr_off(c, q), 16 values of
      // padding per 256 as in the row buffer
#pragma unroll
      for (int c = 0; c < NT; ++c) {
        if (c * kTile >= K_w) break;  // uniform
        if constexpr (RC == 3) {
          // elements b, 4+b, 8+b, 12+b: positions 256 b + 4 lane + 0..3
#pragma unroll
          for (int b = 0; b < 4; ++b)
            *(v2u*)(slice + wlr_off(c, 256 * b + 4 * lane)) = v2u{zs[c][2 * b], zs[c][2 * b + 1]};
        } else {
          // element j: position 256 (lane / 16) + 16 j + lane % 16
          const int q0 = 256 * (lane >> 4) + (lane & 15);
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            *(u16*)(slice + wlr_off(c, q0 + 32 * i)) = (u16)zs[c][i];
            *(u16*)(slice + wlr_off(c, q0 + 32 * i + 16)) = (u16)(zs[c][i] >> 16);
          }
        }
      }
    }
    __builtin_amdgcn_s_setprio(0);
    if constexpr (kDma) {
      if (next < M) stage_row(next);  // every exchange read of this row has returned
    }
    // ---- row scale: RN_dt is monotone, so max |RN_dt(z)| = RN_dt(max |z|)
    amax = wave_max_nonneg(amax);
    if ((t & 63) == 0) red[t >> 6] = amax;
    __syncthreads();
    float mr = red[0];
#pragma unroll
    for (int w = 1; w < TH / 64; ++w) mr = __builtin_fmaxf(mr, red[w]);
    const float m = round_to_dt<DT>(mr);
    const float s = quant_scale(m);
    const float rcp_s = 1.0f / s;
    if (t == 0) s_out[row] = s;

    // ---- gather + quantize + store 16 codes per run
    int8_t* qrow = q_out + (int64_t)row * ldq;
#pragma unroll
    for (int c = 0; c < NT; ++c) {
      if (c * kTile >= K_w) break;  // uniform
      const int o0 = 16 * (t + TH * c);
      float vv[16];
      if (has_perm) {
        const char* rb = (const char*)rowbuf;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          vv[2 * i] = bits16_f32<DT>(*(const u16*)(rb + (po[PLAIN ? 0 : c][i] & 0xffffu)));
          vv[2 * i + 1] = bits16_f32<DT>(*(const u16*)(rb + (po[PLAIN ? 0 : c][i] >> 16)));
        }
      } else if constexpr (WLR) {
        // this lane's 16 consecutive positions are wave-local 16 lane .. 16 lane + 15
        const char* wl = slice + wlr_off(c, 16 * lane);
        unpack8<DT>(*(const v4u*)wl, vv);
        unpack8<DT>(*(const v4u*)(wl + 16), vv + 8);
      } else {
        unpack8<DT>(*(const v4u*)(rowbuf + rbaddr(o0)), vv);
        unpack8<DT>(*(const v4u*)(rowbuf + rbaddr(o0) + 8), vv + 8);
      }
      const v4u codes = quant16(vv, s, rcp_s);
      if (o0 < K_w) *(v4u*)(qrow + o0) = codes;
      __builtin_amdgcn_sched_barrier(0);  // one run at a time keeps the register footprint small
    }
  }
}

// Plain per-token quantization (no rotation, factors or perm), one wave per
// row: the whole row is loaded at once (16 bytes per lane per 512 values),
// unpacked, reduced to the abs-max across the wave, then quantized 8 codes per
// lane per run.
template <int DT, int MAXCH>
__global__ __launch_bounds__(kThreads) void quant_wave_kernel(
    const u16* __restrict__ x, int64_t ldx, int M, int K, int8_t* __restrict__ q_out, int64_t ldq,
    float* __restrict__ s_out) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (row >= M) return;  // wave-uniform
  const u16* xrow = x + (int64_t)row * ldx;
  const int nch = (K + 511) >> 9;  // 512-value chunks (uniform); only the last may be partial
  // Up to 8 chunks the early-exit loops keep the row in a few registers;
  // wider rows use uniform guards instead, so every array index stays a
  // compile-time constant and the row is not demoted to scratch memory.
  v4u a[MAXCH];
  float m = 0.0f;
  if constexpr (MAXCH <= 8) {
#pragma unroll
    for (int i = 0; i < MAXCH; ++i) {
      if (i >= nch) break;
      const int e = min((i * 64 + lane) * 8, K - 8);
      a[i] = *(const v4u*)(xrow + e);
    }
#pragma unroll
    for (int i = 0; i < MAXCH; ++i) {
      if (i >= nch) break;
      float v[8];
      unpack8<DT>(a[i], v);
#pragma unroll
      for (int k = 0; k < 8; ++k) m = __builtin_fmaxf(m, __builtin_fabsf(v[k]));
    }
  } else {
#pragma unroll
    for (int i = 0; i < MAXCH; ++i) {
      a[i] = v4u{0, 0, 0, 0};
      if (i < nch) {
        const int e = min((i * 64 + lane) * 8, K - 8);
        a[i] = *(const v4u*)(xrow + e);
      }
    }
#pragma unroll
    for (int i = 0; i < MAXCH; ++i) {
      if (i < nch) {
        float v[8];
        unpack8<DT>(a[i], v);
#pragma unroll
        for (int k = 0; k < 8; ++k) m = __builtin_fmaxf(m, __builtin_fabsf(v[k]));
      }
    }
  }
  m = wave_max_nonneg(m);
  const float s = quant_scale(m);
  const float rcp_s = 1.0f / s;
  if (lane == 0) s_out[row] = s;
  int8_t* qrow = q_out + (int64_t)row * ldq;
  auto quant_chunk = [&](int i) {
    const int e = (i * 64 + lane) * 8;
    float v[8];
    unpack8<DT>(a[i], v);
    const uint32_t w0 = pack4_lo_bytes(quant_code_mk(v[0], s, rcp_s), quant_code_mk(v[1], s, rcp_s),
                                       quant_code_mk(v[2], s, rcp_s), quant_code_mk(v[3], s, rcp_s));
    const uint32_t w1 = pack4_lo_bytes(quant_code_mk(v[4], s, rcp_s), quant_code_mk(v[5], s, rcp_s),
                                       quant_code_mk(v[6], s, rcp_s), quant_code_mk(v[7], s, rcp_s));
    // streaming stores (measured 9.5 -> 8.3 us at 4096 x 3072; the same for
    // the rotating prep's codes gained nothing)
    if (e < K) __builtin_nontemporal_store(v2u{w0, w1}, (v2u*)(qrow + e));
  };
  if constexpr (MAXCH <= 8) {
#pragma unroll
    for (int i = 0; i < MAXCH; ++i) {
      if (i >= nch) break;
      quant_chunk(i);
    }
  } else {
#pragma unroll
    for (int i = 0; i < MAXCH; ++i)
      if (i < nch) quant_chunk(i);
  }
}

// Persistent grid: resident workgroups per CU (queried once per kernel
// instantiation -- KERN is a template argument, so each instantiation keeps
// its own cached occupancy) times the CUs of the current device.
template <auto KERN>
int persistent_grid(int threads, int64_t M) {
  static thread_local int per_cu = 0;
  if (per_cu == 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, KERN, threads, 0) != hipSuccess || n <= 0) n = 1;
    per_cu = n;
  }
  const int64_t g = (int64_t)per_cu * ic_num_cus();
  return (int)(M < g ? M : g);
}

template <int DT, int LOG4R, int NT, int VAR, int TH = kThreads, int NORM = 0>
hipError_t launch_fast_t(const ic_rotq_args& a, hipStream_t st) {
  constexpr auto kern = rq_fast_kernel<DT, LOG4R, NT, VAR, TH, NORM>;
  const int64_t K_r = LOG4R == 0 ? a.K_in : ((a.K_in + a.rot_size - 1) / a.rot_size) * a.rot_size;
  kern<<<dim3(persistent_grid<kern>(TH, a.M)), dim3(TH), 0, st>>>(
      (const u16*)a.x, a.ldx, (int)a.M, (int)a.K_in, (int)K_r, a.sr_rcp, a.sr_f, (int)a.K_w, a.perm,
      a.q_out, a.ldq, a.s_out, a.nw, a.nb, a.eps);
  return hipGetLastError();
}

template <int DT, int LOG4R, int VAR, int NORM = 0>
hipError_t launch_fast_nt(const ic_rotq_args& a, hipStream_t st) {
  if constexpr (LOG4R == 5) {
    // five one-block waves cover 4097..5120 values in one tile (Wan's 5120
    // would otherwise take two 4096-tiles, 37.5 % of them padding)
    if (a.K_w > kTile && a.K_w <= 320 * 16) return launch_fast_t<DT, LOG4R, 1, VAR, 320, NORM>(a, st);
    // seven one-block waves, two tiles: 12289..14336 values (Wan's FFN-down
    // 14336 instead of four 4096-tiles; ~99 KB of LDS, one workgroup per CU)
    if (a.K_w > 3 * kTile && a.K_w <= 2 * 448 * 16) return launch_fast_t<DT, LOG4R, 2, VAR, 448, NORM>(a, st);
  }
  if constexpr (LOG4R >= 3 && LOG4R <= 5) {
    // one tile of twelve waves for 8193..12288 values (Flux's 12288): the
    // per-thread constants of one tile instead of three
    if (a.K_w > 2 * kTile && a.K_w <= 768 * 16) return launch_fast_t<DT, LOG4R, 1, VAR, 768, NORM>(a, st);
    // two tiles of eight waves for 12289..16384 (Flux's single-block 15360)
    if (a.K_w > 3 * kTile) return launch_fast_t<DT, LOG4R, 2, VAR, 512, NORM>(a, st);
  }
  if constexpr (LOG4R <= 5) {
    // three-wave workgroups where their tile fits the row more tightly
    // (3072: one full tile instead of 3/4 of one; 4097..6144: two)
    constexpr int T3 = 192 * 16;
    if (a.K_w <= T3 && a.K_w > kTile / 2) return launch_fast_t<DT, LOG4R, 1, VAR, 192, NORM>(a, st);
    if (a.K_w > kTile && a.K_w <= 2 * T3) return launch_fast_t<DT, LOG4R, 2, VAR, 192, NORM>(a, st);
  }
  if (a.K_w <= kTile) return launch_fast_t<DT, LOG4R, 1, VAR, kThreads, NORM>(a, st);
  if (a.K_w <= 2 * kTile) return launch_fast_t<DT, LOG4R, 2, VAR, kThreads, NORM>(a, st);
  if (a.K_w <= 3 * kTile) return launch_fast_t<DT, LOG4R, 3, VAR, kThreads, NORM>(a, st);
  return launch_fast_t<DT, LOG4R, 4, VAR, kThreads, NORM>(a, st);
}

// VAR must match the arguments (the per-dtype dispatcher routes on them).
template <int DT, int VAR, int NORM = 0>
hipError_t launch_fast(const ic_rotq_args& a, hipStream_t st) {
  if (NORM == 0 && VAR == kRqPlain && a.rot_size == 0 && a.K_w == a.K_in && a.K_in <= 32 * 512) {
    const unsigned grid = (unsigned)((a.M + 3) / 4);
    if (a.K_in <= 8 * 512)
      quant_wave_kernel<DT, 8><<<grid, kThreads, 0, st>>>((const u16*)a.x, a.ldx, (int)a.M, (int)a.K_in, a.q_out, a.ldq, a.s_out);
    else if (a.K_in <= 16 * 512)
      quant_wave_kernel<DT, 16><<<grid, kThreads, 0, st>>>((const u16*)a.x, a.ldx, (int)a.M, (int)a.K_in, a.q_out, a.ldq, a.s_out);
    else
      quant_wave_kernel<DT, 32><<<grid, kThreads, 0, st>>>((const u16*)a.x, a.ldx, (int)a.M, (int)a.K_in, a.q_out, a.ldq, a.s_out);
    return hipGetLastError();
  }
  switch (a.rot_size) {
    case 0: return launch_fast_nt<DT, 0, VAR, NORM>(a, st);
    case 16: return launch_fast_nt<DT, 2, VAR, NORM>(a, st);
    case 64: return launch_fast_nt<DT, 3, VAR, NORM>(a, st);
    case 256: return launch_fast_nt<DT, 4, VAR, NORM>(a, st);
    case 1024: return launch_fast_nt<DT, 5, VAR, NORM>(a, st);
    case 4096: return launch_fast_nt<DT, 6, VAR, NORM>(a, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace
