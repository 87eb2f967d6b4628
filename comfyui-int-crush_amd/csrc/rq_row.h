// One activation row's preparation and per-token INT8 quantization by a
// 256-thread workgroup, in phases shared by the generic prep kernel
// (rotate_quant.hip) and the single-launch prep + GEMV (gemv_prep.h):
//
//   smoothrot_divide16   SmoothRot divide of 16 positions       (_ops.py:347-350)
//   rotate_tile          block Hadamard of one 4096-position tile in fp64
//                        butterflies, rounded once to the type   (_quant_utils.py:117-147)
//   publish_row          the rotated row, natural order, to LDS (zero pad to K_w, _ops.py:355-358)
//   gather16             PermuQuant gather + old-SmoothQuant divide + abs-max
//                                                               (_ops.py:360-363, :529-533)
//   row_scale            s = max(m, 1e-8) / 127 over the row    (triton_quantize.py:133-135)
//   store_codes16        q = trunc(v/s +- 0.5) clamped           (triton_quantize.py:136-146)
//
// LDS: tbuf (kTbufDoubles doubles, the transpose buffer, reused as the row
// buffer), red (4 floats), xred (kXredWords words, bf16 rows with R = 4096).
#pragma once
#include "rq_common.h"

namespace rq {

constexpr int kTbufDoubles = kTile / 16 * kPadStride;  // 36 KB
constexpr int kXredWords = 2 * (kThreads / 64);

// Register layout class of the rotated values (tile_pos): 0 for no rotation
// and R = 16, 1 for R = 64 / 256, 2 for R = 1024 / 4096.
template <int LOG4R> constexpr int rot_class() { return LOG4R <= 2 ? 0 : (LOG4R <= 4 ? 1 : 2); }

// xs[j] = RN_dt(xs[j] / f[p0 + j]) for positions below K_in; rc holds
// RN32(1/f) of the same positions, sr_f is read on the divide's slow path.
template <int DT> IC_DEV void smoothrot_divide16(float* xs, const float* rc, const float* sr_f, int p0, int K_in) {
#pragma unroll
  for (int j = 0; j < 16; ++j)
    if (p0 + j < K_in) xs[j] = div_round_dt<DT>(xs[j], rc[j], sr_f, p0 + j);
}

// Block Hadamard H_R = (H4/2)^{(x)k}, R = 4^LOG4R, of the tile that starts at
// row position base.  xs: this thread's 16 consecutive positions base + 16t
// .. (after the divide; zero past K_in).  The radix-4 butterflies act on the
// base-4 digits of the in-block index: digits 0-1 in registers, 2-3 after one
// LDS transpose among 16 threads, 4-5 after a second among 256.  val[j]
// receives the value at tile position tile_pos<rot_class>(t, j) rounded once
// to DT (exact fp64 sums for fp16 rows); positions at or past K_r, the rotated
// width, are the zero pad.
template <int DT, int LOG4R>
IC_DEV void rotate_tile(float* xs, double* tbuf, uint32_t* xred, int base, int K_r, float* val) {
  const int t = threadIdx.x;
  if constexpr (DT == IC_DTYPE_BF16 && LOG4R >= 2) bf16_flush_small<LOG4R, kThreads>(xs, xred);
  double v[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) v[j] = (double)xs[j];
  if constexpr (LOG4R >= 2) { stage_lo(v); stage_hi(v); }
  if constexpr (LOG4R >= 3) {
    __syncthreads();  // previous users of tbuf are done
#pragma unroll
    for (int j = 0; j < 16; ++j) tbuf[tslot(16 * t + j)] = v[j];
    __syncthreads();
    const int g = t >> 4, l = t & 15;
#pragma unroll
    for (int h = 0; h < 16; ++h) v[h] = tbuf[tslot(256 * g + 16 * h + l)];
    stage_lo(v);
    if constexpr (LOG4R >= 4) stage_hi(v);
    if constexpr (LOG4R >= 5) {
#pragma unroll
      for (int h = 0; h < 16; ++h) tbuf[tslot(256 * g + 16 * h + l)] = v[h];
      __syncthreads();
#pragma unroll
      for (int gg = 0; gg < 16; ++gg) v[gg] = tbuf[tslot(256 * gg + t)];
      stage_lo(v);
      if constexpr (LOG4R >= 6) stage_hi(v);
    }
  }
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int p = base + tile_pos<rot_class<LOG4R>()>(t, j);
    val[j] = p < K_r ? round_f64_to_dt<DT>(v[j]) : 0.0f;
  }
}

// The prepared row in natural order (16-bit values, or f32 for f32 rows) to
// rowbuf, the tbuf area, for the gather; positions up to K_w.  Barriers on
// both sides: the previous users of tbuf are done before, every value is
// visible after.
template <int DT, int LOG4R, int MAXT>
IC_DEV void publish_row(const float (&val)[MAXT][16], int ntiles, int K_w, char* rowbuf) {
  const int t = threadIdx.x;
  __syncthreads();
#pragma unroll
  for (int tile = 0; tile < MAXT; ++tile) {
    if (tile >= ntiles) break;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int p = tile * kTile + tile_pos<rot_class<LOG4R>()>(t, j);
      if (p < K_w) {
        if constexpr (DT != IC_DTYPE_F32) ((u16*)rowbuf)[p] = f32_bits16<DT>(val[tile][j]);
        else ((float*)rowbuf)[p] = val[tile][j];
      }
    }
  }
  __syncthreads();
}

// Output positions o0 .. o0+15 (below K_w): out[j] = rowbuf[src[j]], divided
// by the old-SmoothQuant factor when has_sm (smr: RN32(1/f) of the same
// positions); returns the running abs-max m over them.  A malformed perm entry
// reads position 0 instead of leaving the row.
template <int DT>
IC_DEV float gather16(const char* rowbuf, const int* src, bool has_sm, const float* smr, const float* sm_f, int o0,
                      int K_w, float* out, float m) {
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int o = o0 + j;
    float vv = 0.0f;
    if (o < K_w) {
      const int sidx = (unsigned)src[j] < (unsigned)K_w ? src[j] : 0;
      if constexpr (DT != IC_DTYPE_F32) vv = bits16_f32<DT>(((const u16*)rowbuf)[sidx]);
      else vv = ((const float*)rowbuf)[sidx];
      if (has_sm) vv = div_round_dt<DT>(vv, smr[j], sm_f, o);
    }
    out[j] = vv;
    m = __builtin_fmaxf(m, __builtin_fabsf(vv));
  }
  return m;
}

// The row's scale from every thread's abs-max m (one barrier; red: 4 floats).
IC_DEV float row_scale(float m, float* red) {
  const int t = threadIdx.x;
  m = wave_max(m);
  if ((t & 63) == 0) red[t >> 6] = m;
  __syncthreads();
  m = __builtin_fmaxf(__builtin_fmaxf(red[0], red[1]), __builtin_fmaxf(red[2], red[3]));
  return quant_scale(m);
}

// Codes of the 16 values of output positions o0 .. (those below K_w), rs =
// RN64(1/s), to qrow (global memory or LDS).
IC_DEV void store_codes16(const float* v, double rs, int8_t* qrow, int o0, int K_w) {
  uint32_t w[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    uint32_t packed = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int code = quant_code(v[4 * d + b], rs);
      packed |= ((uint32_t)code & 0xffu) << (8 * b);
    }
    w[d] = packed;
  }
  if (o0 + 16 <= K_w && ((((uintptr_t)(qrow + o0)) & 15) == 0)) {
    *(v4u*)(qrow + o0) = v4u{w[0], w[1], w[2], w[3]};
  } else {
    for (int j = 0; j < 16 && o0 + j < K_w; ++j) qrow[o0 + j] = (int8_t)(w[j >> 2] >> (8 * (j & 3)));
  }
}

}  // namespace rq
