// INT8 x INT8 -> INT32 MFMA GEMM with fused dequant epilogue (gfx950).
//
//   out[m, n] = f32(acc[m, n]) * (s_a[m] * s_w[n]) + bias[n]                (per-row weight scale)
//   out[m, n] = (sum_g f32(acc_g[m, n]) * s_w[n, g]) * s_a[m] + bias[n]     (per-group weight scale)
//
// A = activation codes [M, K] int8, K-major.  B = weights [N, K], K-major, as
// int8 (W8A8, triton_int8_gemm.py:46-132) or as packed INT4 nibbles (W4A8,
// triton_w4a8_gemm.py:40-108 plus the unpack of triton_int4_to_int8_unpack.py:26-52,
// here fused into the global->LDS copy so the unpacked weight never reaches HBM).
//
// Tiling: 256 threads = 4 waves in a 2x2 grid; each wave owns a (BM/2)x(BN/2)
// sub-tile built from v_mfma_i32_32x32x32_i8 tiles.  K advances 64 bytes per
// stage through a double-buffered LDS ring whose 16-byte chunks are XOR
// swizzled by row to keep ds_read_b128 fragment loads free of bank conflicts.
// INT4 nibbles are expanded to 16*q (int8) with two masks and a byte permute;
// the factor 16 is removed exactly in the epilogue (power-of-two scaling).
#include <type_traits>

#include "ic_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kRowBytes = 64;  // bytes of K per LDS row per stage

IC_DEV int lds_off(int row, int chunk) { return row * kRowBytes + ((chunk ^ ((row >> 1) & 3)) << 4); }

// 8 INT4 nibbles (low nibble = even k) -> 8 int8 values 16*q in natural k order.
IC_DEV void unpack8_x16(uint32_t P, uint32_t& w0, uint32_t& w1) {
  const uint32_t lo = (P << 4) & 0xf0f0f0f0u;  // bytes: 16*q[k=0,2,4,6]
  const uint32_t hi = P & 0xf0f0f0f0u;         // bytes: 16*q[k=1,3,5,7]
  w0 = __builtin_amdgcn_perm(hi, lo, 0x05010400u);  // q0 q1 q2 q3
  w1 = __builtin_amdgcn_perm(hi, lo, 0x07030602u);  // q4 q5 q6 q7
}

// Logical tile id for hardware block id b.  Consecutive block ids are spread
// round-robin over the 8 XCDs; renumber so each XCD works on a contiguous run
// of logical tiles, then walk the run in GROUP_M-row bands so neighbouring
// tiles share A rows and B columns in that XCD's L2.
IC_DEV void tile_coords(int b, int nb, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int xcd = b & 7, local = b >> 3;
  const int per = nb >> 3, rem = nb & 7;
  const int L = xcd < rem ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
  constexpr int GM = 8;
  const int in_group = GM * tiles_n;
  const int group = L / in_group;
  const int first_m = group * GM;
  const int gsize = min(tiles_m - first_m, GM);
  const int r = L - group * in_group;
  tm = first_m + r % gsize;
  tn = r / gsize;
}

template <int BM, int BN, bool INT4, int GS, int OUT_DT, bool ACC_OUT>
__global__ __launch_bounds__(kThreads, 1) void gemm_i8_kernel(
    const int8_t* __restrict__ A, int64_t lda, const uint8_t* __restrict__ B, int64_t ldb,
    const float* __restrict__ s_a, const float* __restrict__ s_w, int G,
    const void* __restrict__ bias, int bias_dt, void* __restrict__ C, int64_t ldc, int M, int N,
    int K, int32_t* __restrict__ acc_out) {
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int A_CH = BM * 4 / kThreads;                      // 16-byte A chunks per thread
  constexpr int B_CH = INT4 ? BN * 2 / kThreads : BN * 4 / kThreads;
  constexpr int STAGE = (BM + BN) * kRowBytes;
  static_assert(TM >= 1 && TN >= 1 && A_CH >= 1 && B_CH >= 1, "tile too small");
  static_assert(GS == 0 || GS == 128, "group size");

  extern __shared__ __attribute__((aligned(16))) char smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wr = wave >> 1, wc = wave & 1;
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int tm, tn;
  tile_coords(blockIdx.x, tiles_m * tiles_n, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int KT = K / 64;

  v4u ra[A_CH], rb[B_CH];
  auto gload = [&](int kt) {
    const int k0 = kt * 64;
#pragma unroll
    for (int c = 0; c < A_CH; ++c) {
      const int q = tid + kThreads * c;
      const int row = min(m0 + (q >> 2), M - 1);
      ra[c] = *(const v4u*)(A + (int64_t)row * lda + k0 + (q & 3) * 16);
    }
#pragma unroll
    for (int c = 0; c < B_CH; ++c) {
      const int q = tid + kThreads * c;
      if constexpr (INT4) {
        const int row = min(n0 + (q >> 1), N - 1);
        rb[c] = *(const v4u*)(B + (int64_t)row * ldb + (k0 >> 1) + (q & 1) * 16);
      } else {
        const int row = min(n0 + (q >> 2), N - 1);
        rb[c] = *(const v4u*)(B + (int64_t)row * ldb + k0 + (q & 3) * 16);
      }
    }
  };
  auto sstore = [&](int buf) {
    char* sA = smem + buf * STAGE;
    char* sB = sA + BM * kRowBytes;
#pragma unroll
    for (int c = 0; c < A_CH; ++c) {
      const int q = tid + kThreads * c;
      *(v4u*)(sA + lds_off(q >> 2, q & 3)) = ra[c];
    }
#pragma unroll
    for (int c = 0; c < B_CH; ++c) {
      const int q = tid + kThreads * c;
      if constexpr (INT4) {
        const int row = q >> 1, h = q & 1;
        uint32_t w[8];
        unpack8_x16(rb[c].x, w[0], w[1]);
        unpack8_x16(rb[c].y, w[2], w[3]);
        unpack8_x16(rb[c].z, w[4], w[5]);
        unpack8_x16(rb[c].w, w[6], w[7]);
        *(v4u*)(sB + lds_off(row, 2 * h)) = v4u{w[0], w[1], w[2], w[3]};
        *(v4u*)(sB + lds_off(row, 2 * h + 1)) = v4u{w[4], w[5], w[6], w[7]};
      } else {
        *(v4u*)(sB + lds_off(q >> 2, q & 3)) = rb[c];
      }
    }
  };

  v16i acc[TM][TN];
  v16f facc[TM][TN];
  (void)facc;
  if constexpr (GS == 0) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = v16i{};
  } else {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) { facc[i][j] = v16f{}; acc[i][j] = v16i{}; }
  }

  // One 64-byte stage: two K-steps of 32.  ZERO_FIRST starts a fresh group
  // accumulator (MFMA with a zero addend) instead of accumulating.
  auto compute = [&](int buf, auto zero_first) {
    constexpr bool ZF = decltype(zero_first)::value;
    const char* sA = smem + buf * STAGE;
    const char* sB = sA + BM * kRowBytes;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      v4i a[TM], b[TN];
      const int ch = 2 * ks + (lane >> 5);
#pragma unroll
      for (int i = 0; i < TM; ++i) a[i] = *(const v4i*)(sA + lds_off(wr * WM + i * 32 + (lane & 31), ch));
#pragma unroll
      for (int j = 0; j < TN; ++j) b[j] = *(const v4i*)(sB + lds_off(wc * WN + j * 32 + (lane & 31), ch));
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          if (ZF && ks == 0) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], v16i{}, 0, 0, 0);
          else acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    }
  };

  // Output coordinates of accumulator element r of tile (i, j) for this lane.
  auto out_row = [&](int i, int r) { return m0 + wr * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); };
  auto out_col = [&](int j) { return n0 + wc * WN + j * 32 + (lane & 31); };

  // Per-group fold: facc += f32(acc_g) * s_w[n, g] (16*acc_g with s_w/16 for INT4).
  auto fold = [&](int g) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = min(out_col(j), N - 1);
      float sw = s_w[(int64_t)n * G + g];
      if constexpr (INT4) sw *= 0.0625f;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        if constexpr (ACC_OUT) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int m = out_row(i, r), nn = out_col(j);
            if (m < M && nn < N) acc_out[((int64_t)g * M + m) * N + nn] = INT4 ? (acc[i][j][r] >> 4) : acc[i][j][r];
          }
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) facc[i][j][r] = __builtin_fmaf((float)acc[i][j][r], sw, facc[i][j][r]);
      }
    }
  };

  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    if (kt + 1 < KT) gload(kt + 1);
    if constexpr (GS == 128) {
      if ((kt & 1) == 0) compute(kt & 1, std::true_type{});
      else { compute(kt & 1, std::false_type{}); fold(kt >> 1); }
    } else {
      compute(kt & 1, std::false_type{});
    }
    if (kt + 1 < KT) sstore((kt + 1) & 1);
    __syncthreads();
  }

  // ---- epilogue
  if constexpr (ACC_OUT && GS == 0) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = out_row(i, r), n = out_col(j);
          if (m < M && n < N) acc_out[(int64_t)m * N + n] = INT4 ? (acc[i][j][r] >> 4) : acc[i][j][r];
        }
  }
  if (C == nullptr) return;
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int n = out_col(j);
    const int nc = min(n, N - 1);
    const float b = bias != nullptr ? ld_any_f32(bias, bias_dt, nc) : 0.0f;
    const float sw = GS == 0 ? s_w[nc] : 0.0f;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = out_row(i, r);
        if (m >= M || n >= N) continue;
        float v;
        if constexpr (GS == 0) {
          float a = (float)acc[i][j][r];
          if constexpr (INT4) a *= 0.0625f;
          v = a * (s_a[m] * sw);
        } else {
          v = facc[i][j][r] * s_a[m];
        }
        if (bias != nullptr) v = v + b;
        st_from_f32<OUT_DT>(C, (int64_t)m * ldc + n, v);
      }
  }
}

// Shape-generic fallback (any K, any alignment): one thread per output, exact
// int32 accumulation; same epilogue arithmetic as the MFMA kernel.
template <bool INT4, int OUT_DT>
__global__ __launch_bounds__(256) void gemm_i8_generic_kernel(
    const int8_t* __restrict__ A, int64_t lda, const uint8_t* __restrict__ B, int64_t ldb,
    const float* __restrict__ s_a, const float* __restrict__ s_w, int G, int gsize,
    const void* __restrict__ bias, int bias_dt, void* __restrict__ C, int64_t ldc, int M, int N,
    int K, int32_t* __restrict__ acc_out) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  const int m = blockIdx.y;
  if (n >= N || m >= M) return;
  const int8_t* a = A + (int64_t)m * lda;
  const uint8_t* b = B + (int64_t)n * ldb;
  float facc = 0.0f;
  int acc = 0;
  for (int k = 0; k < K; ++k) {
    int w;
    if constexpr (INT4) {
      const int nib = (b[k >> 1] >> (4 * (k & 1))) & 0xf;
      w = nib >= 8 ? nib - 16 : nib;
    } else {
      w = (int8_t)b[k];
    }
    acc += (int)a[k] * w;
    if (G > 1 && ((k + 1) % gsize == 0 || k + 1 == K)) {
      const int g = k / gsize;
      if (acc_out) acc_out[((int64_t)g * M + m) * N + n] = acc;
      facc = __builtin_fmaf((float)acc, s_w[(int64_t)n * G + g], facc);
      acc = 0;
    }
  }
  if (G <= 1 && acc_out) acc_out[(int64_t)m * N + n] = acc;
  if (C == nullptr) return;
  float v = G > 1 ? facc * s_a[m] : (float)acc * (s_a[m] * s_w[n]);
  if (bias != nullptr) v = v + ld_any_f32(bias, bias_dt, n);
  st_from_f32<OUT_DT>(C, (int64_t)m * ldc + n, v);
}

struct GemmArgs {
  const int8_t* A; int64_t lda; const uint8_t* B; int64_t ldb;
  const float* s_a; const float* s_w; int G;
  const void* bias; int bias_dt; void* C; int out_dt; int64_t ldc; int M, N, K;
  int32_t* acc_out; bool int4;
};

template <int BM, int BN, bool INT4, int GS, int OUT_DT, bool ACC>
hipError_t launch_mfma(const GemmArgs& g, hipStream_t st) {
  const int tiles = ((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
  const size_t shm = 2 * (BM + BN) * kRowBytes;
  auto kern = gemm_i8_kernel<BM, BN, INT4, GS, OUT_DT, ACC>;
  static bool attr_set = false;  // idempotent attribute; benign if raced
  if (!attr_set) {
    (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
    attr_set = true;
  }
  kern<<<dim3(tiles), dim3(kThreads), shm, st>>>(g.A, g.lda, g.B, g.ldb, g.s_a, g.s_w, g.G, g.bias,
                                                  g.bias_dt, g.C, g.ldc, g.M, g.N, g.K, g.acc_out);
  return hipGetLastError();
}

template <bool INT4, int GS, int OUT_DT, bool ACC>
hipError_t pick_tile(const GemmArgs& g, hipStream_t st) {
  if constexpr (GS == 0) {
    if (g.M >= 256 && g.N >= 256) return launch_mfma<256, 256, INT4, GS, OUT_DT, ACC>(g, st);
    return launch_mfma<128, 128, INT4, GS, OUT_DT, ACC>(g, st);
  } else {
    if (g.M >= 256 && g.N >= 128) return launch_mfma<256, 128, INT4, GS, OUT_DT, ACC>(g, st);
    return launch_mfma<128, 128, INT4, GS, OUT_DT, ACC>(g, st);
  }
}

template <bool INT4, int GS, bool ACC>
hipError_t pick_out(const GemmArgs& g, hipStream_t st) {
  switch (g.out_dt) {
    case IC_DTYPE_F16: return pick_tile<INT4, GS, IC_DTYPE_F16, ACC>(g, st);
    case IC_DTYPE_BF16: return pick_tile<INT4, GS, IC_DTYPE_BF16, ACC>(g, st);
    default: return pick_tile<INT4, GS, IC_DTYPE_F32, ACC>(g, st);
  }
}

template <bool INT4, int OUT_DT>
hipError_t launch_generic_t(const GemmArgs& g, int gsize, hipStream_t st) {
  dim3 grid((unsigned)((g.N + 255) / 256), (unsigned)g.M);
  gemm_i8_generic_kernel<INT4, OUT_DT><<<grid, dim3(256), 0, st>>>(
      g.A, g.lda, g.B, g.ldb, g.s_a, g.s_w, g.G, gsize, g.bias, g.bias_dt, g.C, g.ldc, g.M, g.N, g.K,
      g.acc_out);
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

bool mfma_shape_ok(const GemmArgs& g, int gsize) {
  if (g.K % 64 != 0) return false;
  if (g.G > 1 && gsize != 128) return false;
  if (((uintptr_t)g.A & 15) || ((uintptr_t)g.B & 15) || (g.lda & 15) || (g.ldb & 15)) return false;
  return true;
}

int run_gemm(GemmArgs g, hipStream_t st, const char* who, bool force_generic) {
  if (g.M < 0 || g.N <= 0 || g.K <= 0 || g.lda < g.K || g.ldc < g.N)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: bad shape M=%d N=%d K=%d lda=%lld ldc=%lld", who, g.M,
                        g.N, g.K, (long long)g.lda, (long long)g.ldc);
  if (g.int4 ? (g.ldb * 2 < g.K) : (g.ldb < g.K))
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: weight row stride %lld too small for K=%d", who,
                        (long long)g.ldb, g.K);
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
  if (!force_generic && mfma_shape_ok(g, gsize)) {
    const bool acc = g.acc_out != nullptr;
    if (g.int4) {
      if (g.G > 1) e = acc ? pick_out<true, 128, true>(g, st) : pick_out<true, 128, false>(g, st);
      else e = acc ? pick_out<true, 0, true>(g, st) : pick_out<true, 0, false>(g, st);
    } else {
      if (g.G > 1) e = acc ? pick_out<false, 128, true>(g, st) : pick_out<false, 128, false>(g, st);
      else e = acc ? pick_out<false, 0, true>(g, st) : pick_out<false, 0, false>(g, st);
    }
  } else {
    e = g.int4 ? launch_generic<true>(g, gsize, st) : launch_generic<false>(g, gsize, st);
  }
  if (e != hipSuccess) return ic_set_error(IC_ERR_LAUNCH, "%s: %s", who, hipGetErrorString(e));
  return IC_OK;
}

}  // namespace

extern "C" {

int ic_gemm_w8a8(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const int8_t* w, int64_t N,
                 int64_t ldw, const float* s_a, const float* s_w, const void* bias, int bias_dtype,
                 void* out, int out_dtype, int64_t ldo, void* stream) {
  GemmArgs g{xq, ldx, (const uint8_t*)w, ldw, s_a, s_w, 1, bias, bias_dtype, out, out_dtype, ldo,
             (int)M, (int)N, (int)K, nullptr, false};
  return run_gemm(g, (hipStream_t)stream, "ic_gemm_w8a8", false);
}

int ic_gemm_w4a8(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const uint8_t* w_packed,
                 int64_t N, int64_t ldw, const float* s_w, int64_t num_groups, const float* s_a,
                 const void* bias, int bias_dtype, void* out, int out_dtype, int64_t ldo,
                 void* stream) {
  GemmArgs g{xq, ldx, w_packed, ldw, s_a, s_w, (int)num_groups, bias, bias_dtype, out, out_dtype,
             ldo, (int)M, (int)N, (int)K, nullptr, true};
  return run_gemm(g, (hipStream_t)stream, "ic_gemm_w4a8", false);
}

int ic_gemm_w8a8_acc_i32(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const int8_t* w,
                         int64_t N, int64_t ldw, int32_t* acc, int generic, void* stream) {
  static const float one = 1.0f;
  (void)one;
  GemmArgs g{xq, ldx, (const uint8_t*)w, ldw, nullptr, nullptr, 1, nullptr, 0, nullptr,
             IC_DTYPE_F32, N, (int)M, (int)N, (int)K, acc, false};
  // scales are not read when no output is requested; pass the accumulator as a dummy
  g.s_a = (const float*)acc;
  g.s_w = (const float*)acc;
  return run_gemm(g, (hipStream_t)stream, "ic_gemm_w8a8_acc_i32", generic != 0);
}

int ic_gemm_w4a8_acc_i32(const int8_t* xq, int64_t M, int64_t K, int64_t ldx,
                         const uint8_t* w_packed, int64_t N, int64_t ldw, const float* s_w,
                         int64_t num_groups, int32_t* acc, int generic, void* stream) {
  GemmArgs g{xq, ldx, w_packed, ldw, (const float*)acc, s_w, (int)num_groups, nullptr, 0, nullptr,
             IC_DTYPE_F32, N, (int)M, (int)N, (int)K, acc, true};
  return run_gemm(g, (hipStream_t)stream, "ic_gemm_w4a8_acc_i32", generic != 0);
}

int ic_gemm_w8a8_generic(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const int8_t* w,
                         int64_t N, int64_t ldw, const float* s_a, const float* s_w,
                         const void* bias, int bias_dtype, void* out, int out_dtype, int64_t ldo,
                         void* stream) {
  GemmArgs g{xq, ldx, (const uint8_t*)w, ldw, s_a, s_w, 1, bias, bias_dtype, out, out_dtype, ldo,
             (int)M, (int)N, (int)K, nullptr, false};
  return run_gemm(g, (hipStream_t)stream, "ic_gemm_w8a8_generic", true);
}

}  // extern "C"
