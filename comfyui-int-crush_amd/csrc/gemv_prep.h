// Single-launch small-batch linear on raw activations (M <= 16 tokens): the
// fused preparation + per-token INT8 quantization of ic_rotate_quantize and
// the W8A8 / W4A8 GEMV of gemv_i8.h in one kernel, the single-kernel form of
// the reference's fused quantize + GEMM (kernels/triton_int8_gemm.py:243-389)
// for the small-M use behind _ops.py:443-464 / :493-579.
//
// Every workgroup prepares the M rows itself, with the phases of the generic
// prep kernel (rq_row.h), so codes and scales -- and with them the outputs --
// are bit-identical to ic_rotate_quantize followed by ic_gemv_w*a8.  To keep
// that redundant work small, a workgroup owns several 16-column blocks (at
// most one workgroup per CU), and it issues all of its weight loads before
// the preparation starts, so the weights stream while the rows are prepared.
// One preparation costs each of the four waves about 1700 VALU instructions
// (fp64 butterflies, exact divides and codes); with one 4-wave workgroup per
// CU the weight stream itself is slower than the GEMV's, whose many
// workgroups per CU keep more requests in flight.  At the Flux modulation
// shape this kernel is slower than the two launches it replaces, which
// remain the library's default path; it is the form for callers that want
// a single kernel.
//
// LDS: the prep's transpose / row buffer (36 KB), reused for the block sums
// of the workgroup's column blocks once the codes are written, and the
// [M][K] codes (M * K <= 16 KB).
#pragma once
#include "gemv_i8.h"
#include "rq_row.h"

namespace gemvp {

using namespace rq;

// Arguments of the preparation (as ic_rotate_quantize takes them; K_w is the
// GEMV's K).
struct PrepArgs {
  const void* x;
  int64_t ldx;
  int K_in, K_r;  // input width and rotated width
  const float* sr_rcp;
  const float* sr_f;
  const int32_t* perm;
  const float* sm_rcp;
  const float* sm_f;
};

// Preparation of the M rows into LDS codes (xs) and scales (sa).  NT: the
// 4096-position tiles of a row (K <= 4096: 1, else 2).  The entry points
// admit 16-byte aligned rows, factors and perm with K_in a multiple of 16, so
// each thread's 16 positions are either all inside the row or all past it:
// every preload is one unconditional 16-byte load per 8 (16-bit) or 4
// (32-bit) values, from a clamped address when past the row, and the number
// of loads issued after it is the same on every path (the compiler then waits
// for the preloads without waiting for the weight loads issued after them).
template <int DT, int LOG4R, int NT>
struct PrepCodes {
  static_assert(DT != IC_DTYPE_F32, "16-bit activation rows");
  PrepArgs a;
  int K_w;
  double* tbuf;
  float* red;
  uint32_t* xred;
  float* sa;
  v4u xr[NT][2];  // this thread's 16 input values of the current row, as loaded
  v4u rc[NT][4];  // the bits of their SmoothRot reciprocals (all rows)
  v4u pr[NT][4];  // perm entries of this thread's output positions (all rows)
  v4u sm[NT][4];  // the bits of their old-SmoothQuant reciprocals (all rows)

  IC_DEV int pos0(int tile) const { return tile * kTile + 16 * (int)threadIdx.x; }
  IC_DEV void load_row(int m) {
    const u16* xrow = (const u16*)a.x + (int64_t)m * a.ldx;
#pragma unroll
    for (int tile = 0; tile < NT; ++tile) {
      const u16* p = xrow + min(pos0(tile), a.K_in - 16);
      xr[tile][0] = *(const v4u*)p;
      xr[tile][1] = *(const v4u*)(p + 8);
    }
  }
  // before the first weight loads: these loads then complete without waiting
  // for the weights (vector-memory loads retire in issue order)
  IC_DEV void preload() {
    load_row(0);
#pragma unroll
    for (int tile = 0; tile < NT; ++tile) {
      if (a.sr_rcp != nullptr) {
        const float* p = a.sr_rcp + min(pos0(tile), a.K_in - 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) rc[tile][i] = *(const v4u*)(p + 4 * i);
      }
      if (a.perm != nullptr) {
        const int32_t* p = a.perm + min(pos0(tile), K_w - 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) pr[tile][i] = *(const v4u*)(p + 4 * i);
      }
      if (a.sm_rcp != nullptr) {
        const float* p = a.sm_rcp + min(pos0(tile), K_w - 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) sm[tile][i] = *(const v4u*)(p + 4 * i);
      }
    }
  }
  static IC_DEV void unpack_f32(const v4u (&q)[4], float* o) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[4 * i] = __uint_as_float(q[i].x);
      o[4 * i + 1] = __uint_as_float(q[i].y);
      o[4 * i + 2] = __uint_as_float(q[i].z);
      o[4 * i + 3] = __uint_as_float(q[i].w);
    }
  }
  // Row m (its inputs loaded into xr) to codes xs_row and scale sa[m].
  IC_DEV void prep_row(int m, int8_t* xs_row) {
    const int t = threadIdx.x;
    char* rowbuf = (char*)tbuf;
    float val[NT][16];
#pragma unroll
    for (int tile = 0; tile < NT; ++tile) {
      const int p0 = pos0(tile);
      const bool in_row = p0 < a.K_in;
      float xv[16];
      const uint32_t w[8] = {xr[tile][0].x, xr[tile][0].y, xr[tile][0].z, xr[tile][0].w,
                             xr[tile][1].x, xr[tile][1].y, xr[tile][1].z, xr[tile][1].w};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        xv[2 * i] = in_row ? bits16_f32<DT>((u16)(w[i] & 0xffffu)) : 0.0f;
        xv[2 * i + 1] = in_row ? bits16_f32<DT>((u16)(w[i] >> 16)) : 0.0f;
      }
      if (a.sr_rcp != nullptr && in_row) {
        float r[16];
        unpack_f32(rc[tile], r);
        smoothrot_divide16<DT>(xv, r, a.sr_f, p0, p0 + 16);  // all 16 positions lie in the row
      }
      rotate_tile<DT, LOG4R>(xv, tbuf, xred, tile * kTile, a.K_r, val[tile]);
    }
    publish_row<DT, LOG4R, NT>(val, NT, K_w, rowbuf);
    float mx = 0.0f;
#pragma unroll
    for (int c = 0; c < NT; ++c) {
      const int o0 = 16 * (t + kThreads * c);
      int src[16];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (a.perm != nullptr) {
          src[4 * i] = (int)pr[c][i].x;
          src[4 * i + 1] = (int)pr[c][i].y;
          src[4 * i + 2] = (int)pr[c][i].z;
          src[4 * i + 3] = (int)pr[c][i].w;
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) src[4 * i + j] = o0 + 4 * i + j;
        }
      }
      float smr[16];
      unpack_f32(sm[c], smr);
      mx = gather16<DT>(rowbuf, src, a.sm_rcp != nullptr, smr, a.sm_f, o0, K_w, val[c], mx);
    }
    const float s = row_scale(mx, red);
    const double rs = 1.0 / (double)s;
    if (t == 0) sa[m] = s;
#pragma unroll
    for (int c = 0; c < NT; ++c) {
      const int o0 = 16 * (t + kThreads * c);
      if (o0 < K_w) store_codes16(val[c], rs, xs_row, o0, K_w);
    }
  }
  // Row 0 is peeled: its inputs came with the preloads, so the compiler waits
  // for them alone; later rows load theirs after the weights.
  IC_DEV void fill(int8_t* xs, int M, int K) {
    prep_row(0, xs);
    for (int m = 1; m < M; ++m) {
      load_row(m);
      prep_row(m, xs + (int64_t)m * K);
    }
  }
};

// Weight loads a wave holds at once (128 VGPRs).
template <bool INT4> constexpr int kPrepGemvSteps = INT4 ? 32 : 16;

// One workgroup owns cbs consecutive 16-column blocks (the host picks cbs so
// that there is at most one workgroup per CU where the block sums and loads
// allow: the preparation is done once per workgroup and its VALU work is not
// shared with another workgroup's).  Each wave walks its K blocks of every
// column block in turn (block b = wave + 4u of column block j is step
// f = j * UB + u, F = cbs * UB <= kPrepGemvSteps steps).  All of a wave's
// weight loads are issued before the preparation starts, as the GEMV on INT8
// codes issues its batch: the whole weight slice is in flight while the rows
// are prepared.  Every load is issued (steps past the last reload the last),
// so the compiler's waits before each step count exactly the loads behind
// it.  The sums of all the column blocks stay in LDS; after one barrier the
// workgroup writes every output.
template <bool INT4, int GS, int DT, int LOG4R, int NT>
__global__ __launch_bounds__(gemv::kGT) void prep_gemv_kernel(
    PrepArgs pa, const uint8_t* __restrict__ B, int64_t ldb, const float* __restrict__ s_w, int G,
    const void* __restrict__ bias, int bias_dt, void* __restrict__ C, int out_dt, int64_t ldc, int M, int N, int K,
    int cbs, ic_epi epi) {
  static_assert(kThreads == gemv::kGT, "the prep phases and the GEMV share the workgroup");
  using gemv::kGBK;
  // the prep's transpose / row buffer, then the GEMV's block sums: per
  // column block [K/128][M][16] (GS == 128) or [4][M][16] int32
  __shared__ __attribute__((aligned(16))) double tbuf[kTbufDoubles];
  __shared__ float red[kThreads / 64];
  __shared__ uint32_t xred[kXredWords];
  __shared__ float sa[IC_GEMV_MAX_M];
  extern __shared__ __attribute__((aligned(16))) int8_t xs[];  // [M][K] codes
  int32_t* sacc = (int32_t*)tbuf;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane >> 4, col = lane & 15;
  const int KB = K / kGBK;
  const int UB = (KB + 3) / 4;  // steps of each wave per column block
  const int cb_first = blockIdx.x * cbs;
  const int ncb = min(cbs, (N + 15) / 16 - cb_first);
  const int F = ncb * UB;       // steps of each wave
  const int sacc_cb = (GS == 128 ? KB : 4) * M * 16;  // ints per column block
  const int8_t* arow = xs + (int64_t)min(col, M - 1) * K + 32 * c;

  PrepCodes<DT, LOG4R, NT> prep;
  prep.a = pa;
  prep.K_w = K;
  prep.tbuf = tbuf;
  prep.red = red;
  prep.xred = xred;
  prep.sa = sa;
  prep.preload();  // before the weight loads: waited for without them

  constexpr int kS = kPrepGemvSteps<INT4>;
  v4u pw[kS];
  v4i w1[INT4 ? 1 : kS];
#pragma unroll
  for (int i = 0; i < kS; ++i) {
    const int f = min(i, F - 1);
    const int j = f / UB, b = min(wave + 4 * (f - j * UB), KB - 1);
    const int n = min((cb_first + j) * 16 + col, N - 1);
    const uint8_t* brow = B + (int64_t)n * ldb + (INT4 ? 16 * c : 32 * c);
    if constexpr (INT4) {
      pw[i] = *(const v4u*)(brow + (kGBK / 2) * b);
    } else {
      pw[i] = *(const v4u*)(brow + kGBK * b);
      w1[i] = *(const v4i*)(brow + kGBK * b + 16);
    }
  }

  prep.fill(xs, M, K);
  __syncthreads();
  v4i tot = {0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < kS; ++i) {
    if (i < F) {  // uniform across the wave
      const int j = i / UB, u = i - j * UB, b = wave + 4 * u;
      int32_t* sj = sacc + j * sacc_cb;
      if (b < KB)
        gemv::mma_block<INT4, GS>(b, *(const v4i*)(arow + kGBK * b), *(const v4i*)(arow + kGBK * b + 16), pw[i],
                                  w1[INT4 ? 0 : i], M, c, col, sj, tot);
      if constexpr (GS == 0) {
        if (u == UB - 1) {
          gemv::store_wave_totals(tot, wave, M, c, col, sj);
          tot = v4i{0, 0, 0, 0};
        }
      }
    }
  }
  __syncthreads();
  for (int o = tid; o < ncb * 16 * M; o += kThreads) {
    const int j = o / (16 * M), r = o - j * 16 * M;
    gemv::gemv_output<INT4, GS, gemv::kOutRuntime>(r >> 4, r & 15, sacc + j * sacc_cb, KB, M, (cb_first + j) * 16,
                                                   N, sa, s_w, G, K / G, bias, bias_dt, C, out_dt, ldc, epi);
  }
}

// Host-side launch description (arguments checked by the entry points).
struct PrepGemvLaunch {
  PrepArgs pa;
  int log4r;          // 0 (no rotation) or 2..6
  bool int4, grouped; // INT4 weights; per-128 group scales
  const uint8_t* B;
  int64_t ldb;
  const float* s_w;
  int G;
  const void* bias;
  int bias_dt;
  void* C;
  int out_dt;
  int64_t ldc;
  int M, N, K;
  int cbs;  // 16-column blocks per workgroup
  ic_epi epi;
};

template <bool INT4, int GS, int DT, int LOG4R, int NT>
hipError_t launch_prep_gemv_k(const PrepGemvLaunch& L, hipStream_t st) {
  const int nblk = (L.N + 15) / 16;
  prep_gemv_kernel<INT4, GS, DT, LOG4R, NT><<<dim3((unsigned)((nblk + L.cbs - 1) / L.cbs)), dim3(gemv::kGT),
                                              (size_t)L.M * L.K, st>>>(
      L.pa, L.B, L.ldb, L.s_w, L.G, L.bias, L.bias_dt, L.C, L.out_dt, L.ldc, L.M, L.N, L.K, L.cbs, L.epi);
  return hipGetLastError();
}

template <int DT, int LOG4R, int NT>
hipError_t launch_prep_gemv_w(const PrepGemvLaunch& L, hipStream_t st) {
  if (L.int4 && L.grouped) return launch_prep_gemv_k<true, 128, DT, LOG4R, NT>(L, st);
  if (L.int4) return launch_prep_gemv_k<true, 0, DT, LOG4R, NT>(L, st);
  return launch_prep_gemv_k<false, 0, DT, LOG4R, NT>(L, st);
}

template <int DT, int NT>
hipError_t launch_prep_gemv(const PrepGemvLaunch& L, hipStream_t st) {
  switch (L.log4r) {
    case 0: return launch_prep_gemv_w<DT, 0, NT>(L, st);
    case 2: return launch_prep_gemv_w<DT, 2, NT>(L, st);
    case 3: return launch_prep_gemv_w<DT, 3, NT>(L, st);
    case 4: return launch_prep_gemv_w<DT, 4, NT>(L, st);
    case 5: return launch_prep_gemv_w<DT, 5, NT>(L, st);
    case 6: return launch_prep_gemv_w<DT, 6, NT>(L, st);
  }
  return hipErrorInvalidValue;
}

// rows span kPrepGemvMaxTiles tiles at most: K <= 8192
constexpr int kPrepGemvMaxTiles = 2;

}  // namespace gemvp

// Instantiations, one activation type and tile count per source file
// (gemv_prep_{f16,bf16}_t{1,2}.hip).
hipError_t ic_prep_gemv_f16_t1(const gemvp::PrepGemvLaunch& L, hipStream_t st);
hipError_t ic_prep_gemv_f16_t2(const gemvp::PrepGemvLaunch& L, hipStream_t st);
hipError_t ic_prep_gemv_bf16_t1(const gemvp::PrepGemvLaunch& L, hipStream_t st);
hipError_t ic_prep_gemv_bf16_t2(const gemvp::PrepGemvLaunch& L, hipStream_t st);
