// Small-batch (M <= 16 tokens) quantized linears on gfx950: bandwidth-bound
// GEMV kernels that read every packed weight byte once.
//
// The reference runs every batch size through the tiled GEMM (_ops.py:493-579,
// triton_w4a8_gemm.py:111-169); a 256-row GEMM tile is >90% padding at M = 1
// (Flux modulation layers, CFG batch 2).  Here one 256-thread workgroup owns
// 16 output columns and its four waves split K in blocks of 128:
//
//   W8A8 / W4A8:  two v_mfma_i32_16x16x64_i8 per block on exact int32 block
//                 sums, the tiled GEMM's epilogue formula (body in gemv_i8.h,
//                 shared with the single-launch prep + GEMV of gemv_prep.h)
//   W4A16:        four v_mfma_f32_16x16x32_{f16,bf16} per block on weights
//                 dequantized exactly as RN_dt(q * RN_dt(s)); fp32 partials of
//                 the four waves are added in wave order.
//
// Every lane of a wave reads 16 packed bytes (32 values) of one weight row per
// block, so a wave-wide load covers 16 rows x 64 bytes.  When the M x K
// activations fit 16 KB (M = 1 up to K = 8192 for 16-bit activations) they
// are staged in LDS once per workgroup and read per block from there, so the
// registers hold weights only and more waves keep loads in flight.
#include <type_traits>

#include "dequant4.h"
#include "gemv_i8.h"

namespace {

using gemv::kGT;
using gemv::kGBK;
using gemv::kXlBytes;

typedef _Float16 v8h_t __attribute__((ext_vector_type(8)));
typedef __bf16 v8bf_t __attribute__((ext_vector_type(8)));

// Ints of block sums: grouped (GS = fold block) [K/GS][M][16], per row
// [4][M][16].
constexpr int64_t gemv_sums(int GS, int64_t M, int64_t K) { return (GS ? K / GS : 4) * M * 16; }

template <bool INT4, int GS, int OUT_DT, bool XL>
__global__ __launch_bounds__(kGT) void gemv_i8_kernel(
    const int8_t* __restrict__ A, int64_t lda, const uint8_t* __restrict__ B, int64_t ldb,
    const float* __restrict__ s_a, const float* __restrict__ s_w, int G, int gsize,
    const void* __restrict__ bias, int bias_dt, void* __restrict__ C, int64_t ldc, int M, int N, int K,
    ic_epi epi, W4Sel sel) {
  // the block sums, then with XL the activation codes [M][K]
  extern __shared__ int32_t sacc[];
  int8_t* xs = (int8_t*)(sacc + gemv_sums(GS, M, K));
  gemv::gemv_i8_body<INT4, GS, OUT_DT, XL>(A, lda, B, ldb, s_a, s_w, G, gsize, bias, bias_dt, C, ldc, M, N, K, epi,
                                           sacc, xs, sel);
}

// W4A16 weight dequantization RN_dt(q * RN_dt(s)) of 8 nibbles.
//
// XL: the M x K activations (at most kXlBytes) are first copied into LDS and
// each block's fragments read from there when used.  Held in registers for a
// batch of 8 blocks, they were 4x the weight bytes per lane and 128 VGPRs,
// which left two waves per SIMD and too few weight loads in flight (16.5 us,
// 1.8 TB/s, at the Flux modulation shape; 12.7 us with the staging).  The
// weight scales are staged too (82 -> 71 VGPRs, no per-block division or
// scattered scale load): 11.7 us.
template <int DT, bool XL>
__global__ __launch_bounds__(kGT) void gemv_w4a16_kernel(
    const u16* __restrict__ X, int64_t ldx, const uint8_t* __restrict__ B, int64_t ldb,
    const float* __restrict__ s_w, int G, int gsize, const void* __restrict__ bias, int bias_dt,
    u16* __restrict__ C, int64_t ldc, int M, int N, int K) {
  __shared__ float sacc[4 * 16 * 16];
  // the workgroup's 16 x G weight scales, then (XL) M rows of K activations
  extern __shared__ __attribute__((aligned(16))) float ssc[];
  u16* xs = (u16*)(ssc + ((16 * G + 3) & ~3));
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n0 = blockIdx.x * 16;
  const int c = lane >> 4, col = lane & 15;
  const int n = min(n0 + col, N - 1);
  const int am = min(col, M - 1);
  const int KB = K / kGBK;
  const uint8_t* brow = B + (int64_t)n * ldb + 16 * c;
  const u16* xrow = XL ? xs + (int64_t)am * K + 32 * c : X + (int64_t)am * ldx + 32 * c;
  // The scales of the 16 columns are one contiguous run of s_w (rows n0 ..
  // n0+15); staged once, read per block from LDS.  The lane's 32 values of
  // block b are quarter q = 4b + c of 32 columns, in group q / (gsize / 32),
  // formed as trunc((q + 1/2) / gq) in f32 (exact: q < 2^9, and the half
  // keeps the product clear of the integers).
  auto stage_scales = [&] {
    for (int i = tid; i < 16 * G; i += kGT) {
      const int r = i / G;
      ssc[i] = s_w[(int64_t)min(n0 + r, N - 1) * G + (i - r * G)];
    }
  };
  const float inv_gq = 32.0f / (float)gsize;
  const float* sc_col = ssc + col * G;
  auto scale_of = [&](int b) { return G > 1 ? sc_col[(int)(((float)(4 * b + c) + 0.5f) * inv_gq)] : sc_col[0]; };

  constexpr int kBatch = 8;
  v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
  // One block: four MFMAs on this lane's 32 activations and 32 dequantized weights.
  auto mma_block = [&](int b, const v4u* xq, const v4u& pwu, float svu) {
    const uint32_t p4[4] = {pwu.x, pwu.y, pwu.z, pwu.w};
    const DeqScale d = deq_scale<DT>(svu);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t o[4];
      deq8<DT>(p4[j], d, o);
      const v4u wv = {o[0], o[1], o[2], o[3]};
      const v4u xa = XL ? *(const v4u*)(xrow + kGBK * b + 8 * j) : xq[j];
      if constexpr (DT == IC_DTYPE_F16)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h_t, xa), __builtin_bit_cast(v8h_t, wv), acc, 0, 0, 0);
      else
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf_t, xa), __builtin_bit_cast(v8bf_t, wv), acc, 0, 0, 0);
    }
  };
  if constexpr (XL) {
    // staged first: issuing the first batch of weight loads ahead of the copy
    // measured slower (13.1 against 11.7 us at 1 x 3072 -> 18432), as did
    // holding a batch of weights across it (~20 VGPRs, lower occupancy)
    stage_scales();
    const int per_row = K / 8;  // 16-byte chunks
    for (int i = tid; i < M * per_row; i += kGT) {
      const int r = i / per_row, k8 = i - r * per_row;
      *(v4u*)(xs + (int64_t)r * K + 8 * k8) = *(const v4u*)(X + (int64_t)r * ldx + 8 * k8);
    }
    __syncthreads();
    for (int b0 = wave; b0 < KB; b0 += 4 * kBatch) {
      v4u pw[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int b = b0 + 4 * u;
        if (b < KB) pw[u] = *(const v4u*)(brow + (kGBK / 2) * b);  // uniform across the wave
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int b = b0 + 4 * u;
        if (b >= KB) break;
        mma_block(b, nullptr, pw[u], scale_of(b));
      }
    }
  } else {
    stage_scales();
    __syncthreads();
    for (int b0 = wave; b0 < KB; b0 += 4 * kBatch) {
      v4u xv[kBatch][4], pw[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int b = b0 + 4 * u;
        if (b < KB) {  // uniform across the wave
#pragma unroll
          for (int j = 0; j < 4; ++j) xv[u][j] = *(const v4u*)(xrow + kGBK * b + 8 * j);
          pw[u] = *(const v4u*)(brow + (kGBK / 2) * b);
        }
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int b = b0 + 4 * u;
        if (b >= KB) break;
        mma_block(b, xv[u], pw[u], scale_of(b));
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) sacc[(wave * 16 + 4 * c + i) * 16 + col] = acc[i];
  __syncthreads();
  if (tid >= 16 * M) return;
  const int m = tid >> 4, nl = tid & 15, no = n0 + nl;
  if (no >= N) return;
  float v = ((sacc[(0 * 16 + m) * 16 + nl] + sacc[(1 * 16 + m) * 16 + nl]) + sacc[(2 * 16 + m) * 16 + nl]) +
            sacc[(3 * 16 + m) * 16 + nl];
  if (bias != nullptr) v = v + ld_any_f32(bias, bias_dt, no);
  st_from_f32<DT>(C, (int64_t)m * ldc + no, v);
}

template <bool INT4, int GS, int OUT_DT, bool XL>
hipError_t launch_gemv_i8_t(const int8_t* A, int64_t lda, const uint8_t* B, int64_t ldb, const float* s_a,
                            const float* s_w, int G, const void* bias, int bias_dt, void* C, int64_t ldc,
                            int M, int N, int K, const ic_epi& epi, W4Sel sel, hipStream_t st) {
  auto kern = gemv_i8_kernel<INT4, GS, OUT_DT, XL>;
  const size_t shm = (size_t)gemv_sums(GS, M, K) * 4 + (XL ? (size_t)M * K : 0);
  static unsigned char lds_set[64];  // per device
  if (hipError_t e = ic_set_lds_limit((const void*)kern, 160 * 1024, lds_set)) return e;
  kern<<<dim3((unsigned)((N + 15) / 16)), dim3(kGT), shm, st>>>(A, lda, B, ldb, s_a, s_w, G, K / G, bias, bias_dt,
                                                                C, ldc, M, N, K, epi, sel);
  return hipGetLastError();
}

template <bool INT4, int GS, int OUT_DT>
hipError_t launch_gemv_i8(const int8_t* A, int64_t lda, const uint8_t* B, int64_t ldb, const float* s_a,
                          const float* s_w, int G, const void* bias, int bias_dt, void* C, int64_t ldc,
                          int M, int N, int K, const ic_epi& epi, W4Sel sel, hipStream_t st) {
  if ((int64_t)M * K <= kXlBytes && gemv_sums(GS, M, K) * 4 + (int64_t)M * K <= 160 * 1024)
    return launch_gemv_i8_t<INT4, GS, OUT_DT, true>(A, lda, B, ldb, s_a, s_w, G, bias, bias_dt, C, ldc, M, N, K, epi,
                                                    sel, st);
  return launch_gemv_i8_t<INT4, GS, OUT_DT, false>(A, lda, B, ldb, s_a, s_w, G, bias, bias_dt, C, ldc, M, N, K, epi,
                                                   sel, st);
}

template <bool INT4, int GS>
hipError_t pick_gemv_out(int out_dt, const int8_t* A, int64_t lda, const uint8_t* B, int64_t ldb,
                         const float* s_a, const float* s_w, int G, const void* bias, int bias_dt, void* C,
                         int64_t ldc, int M, int N, int K, const ic_epi& epi, W4Sel sel, hipStream_t st) {
  switch (out_dt) {
    case IC_DTYPE_F16:
      return launch_gemv_i8<INT4, GS, IC_DTYPE_F16>(A, lda, B, ldb, s_a, s_w, G, bias, bias_dt, C, ldc, M, N, K, epi,
                                                    sel, st);
    case IC_DTYPE_BF16:
      return launch_gemv_i8<INT4, GS, IC_DTYPE_BF16>(A, lda, B, ldb, s_a, s_w, G, bias, bias_dt, C, ldc, M, N, K, epi,
                                                     sel, st);
    default:
      return launch_gemv_i8<INT4, GS, IC_DTYPE_F32>(A, lda, B, ldb, s_a, s_w, G, bias, bias_dt, C, ldc, M, N, K, epi,
                                                    sel, st);
  }
}

int check_gemv_common(const char* who, int64_t M, int64_t K, int64_t N, int64_t ldx, int64_t ldo,
                      const void* bias, int bias_dtype) {
  if (M < 0 || M > IC_GEMV_MAX_M)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: M=%lld outside [0, %d]", who, (long long)M, IC_GEMV_MAX_M);
  if (N <= 0 || K <= 0 || ldx < K || ldo < N)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: bad shape N=%lld K=%lld", who, (long long)N, (long long)K);
  if (K % kGBK != 0 || K > IC_GEMV_MAX_K)
    return ic_set_error(IC_ERR_UNSUPPORTED, "%s: K=%lld must be a multiple of %d and <= %d", who, (long long)K,
                        kGBK, IC_GEMV_MAX_K);
  if (bias && bias_dtype != IC_DTYPE_F16 && bias_dtype != IC_DTYPE_BF16 && bias_dtype != IC_DTYPE_F32)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: bias dtype must be f16/bf16/f32", who);
  return IC_OK;
}

}  // namespace

// Grouped W4A8 folds per gcd(group, 128) columns, as the GEMM kernels do.
static int fold_block(int64_t gsize) {
  int64_t a = gsize, b = 128;
  while (b != 0) {
    const int64_t t = a % b;
    a = b;
    b = t;
  }
  return (int)a;
}

// Shared by the GEMM entry points, which route M <= 16 here.
bool ic_gemv_w4a8_groups_ok(int64_t M, int64_t K, int64_t num_groups) {
  if (num_groups == 1) return true;
  if (num_groups < 1 || K % num_groups != 0 || (K / num_groups) % 32 != 0) return false;
  return gemv_sums(fold_block(K / num_groups), M, K) * 4 <= 128 * 1024;
}
// Shared by the GEMM entry points, which route M <= 16 here.
bool ic_gemv_applicable(int64_t M, int64_t K, const void* x, int64_t ldx_bytes, const void* w, int64_t ldw_bytes) {
  return M >= 1 && M <= IC_GEMV_MAX_M && K % kGBK == 0 && K <= IC_GEMV_MAX_K && ((uintptr_t)x & 15) == 0 &&
         ((uintptr_t)w & 15) == 0 && (ldx_bytes & 15) == 0 && (ldw_bytes & 15) == 0;
}

// GEMV bodies with the activation / residual epilogue (the GEMM entry points
// route M <= 16 here with theirs; the C entry points below pass none).
int ic_gemv_w8a8_epi(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const int8_t* w, int64_t N, int64_t ldw,
                     const float* s_a, const float* s_w, const void* bias, int bias_dtype, void* out, int out_dtype,
                     int64_t ldo, const ic_epi& epi, void* stream) {
  const char* who = "ic_gemv_w8a8";
  int rc = check_gemv_common(who, M, K, N, ldx, ldo, bias, bias_dtype);
  if (rc) return rc;
  if (M == 0) return IC_OK;
  if (!xq || !w || !s_a || !s_w || !out) return ic_set_error(IC_ERR_INVALID_ARG, "%s: null pointer", who);
  if (!ic_gemv_applicable(M, K, xq, ldx, w, ldw) || ldw < K)
    return ic_set_error(IC_ERR_UNSUPPORTED, "%s: operands must be 16-byte aligned", who);
  if (out_dtype != IC_DTYPE_F16 && out_dtype != IC_DTYPE_BF16 && out_dtype != IC_DTYPE_F32)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: out dtype must be f16/bf16/f32", who);
  hipError_t e = pick_gemv_out<false, 0>(out_dtype, xq, ldx, (const uint8_t*)w, ldw, s_a, s_w, 1, bias, bias_dtype,
                                         out, ldo, (int)M, (int)N, (int)K, epi, kW4Plain, (hipStream_t)stream);
  if (e != hipSuccess) return ic_set_error(IC_ERR_LAUNCH, "%s: %s", who, hipGetErrorString(e));
  return IC_OK;
}

int ic_gemv_w4a8_epi(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const uint8_t* w_packed, int64_t N,
                     int64_t ldw, const float* s_w, int64_t num_groups, const float* s_a, const void* bias,
                     int bias_dtype, void* out, int out_dtype, int64_t ldo, const ic_epi& epi, void* stream,
                     W4Sel sel) {
  const char* who = "ic_gemv_w4a8";
  int rc = check_gemv_common(who, M, K, N, ldx, ldo, bias, bias_dtype);
  if (rc) return rc;
  if (!ic_gemv_w4a8_groups_ok(M, K, num_groups))
    return ic_set_error(IC_ERR_UNSUPPORTED,
                        "%s: num_groups must be 1 or give groups of a multiple of 32 columns whose %d-column fold "
                        "sums of M x K fit 128 KB", who, num_groups > 1 ? fold_block(K / num_groups) : 0);
  if (M == 0) return IC_OK;
  if (!xq || !w_packed || !s_a || !s_w || !out) return ic_set_error(IC_ERR_INVALID_ARG, "%s: null pointer", who);
  if (!ic_gemv_applicable(M, K, xq, ldx, w_packed, ldw) || ldw * 2 < K)
    return ic_set_error(IC_ERR_UNSUPPORTED, "%s: operands must be 16-byte aligned", who);
  if (out_dtype != IC_DTYPE_F16 && out_dtype != IC_DTYPE_BF16 && out_dtype != IC_DTYPE_F32)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: out dtype must be f16/bf16/f32", who);
  hipStream_t st = (hipStream_t)stream;
  const int fb = num_groups > 1 ? fold_block(K / num_groups) : 0;
  auto go = [&](auto gs_c) {
    return pick_gemv_out<true, decltype(gs_c)::value>(out_dtype, xq, ldx, w_packed, ldw, s_a, s_w, (int)num_groups,
                                                      bias, bias_dtype, out, ldo, (int)M, (int)N, (int)K, epi, sel,
                                                      st);
  };
  hipError_t e = fb == 128 ? go(std::integral_constant<int, 128>{})
                 : fb == 64 ? go(std::integral_constant<int, 64>{})
                 : fb == 32 ? go(std::integral_constant<int, 32>{})
                            : go(std::integral_constant<int, 0>{});
  if (e != hipSuccess) return ic_set_error(IC_ERR_LAUNCH, "%s: %s", who, hipGetErrorString(e));
  return IC_OK;
}

extern "C" {

int ic_gemv_w8a8(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const int8_t* w, int64_t N, int64_t ldw,
                 const float* s_a, const float* s_w, const void* bias, int bias_dtype, void* out, int out_dtype,
                 int64_t ldo, void* stream) {
  return ic_gemv_w8a8_epi(xq, M, K, ldx, w, N, ldw, s_a, s_w, bias, bias_dtype, out, out_dtype, ldo, ic_epi{}, stream);
}

int ic_gemv_w4a8(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const uint8_t* w_packed, int64_t N,
                 int64_t ldw, const float* s_w, int64_t num_groups, const float* s_a, const void* bias,
                 int bias_dtype, void* out, int out_dtype, int64_t ldo, void* stream) {
  return ic_gemv_w4a8_epi(xq, M, K, ldx, w_packed, N, ldw, s_w, num_groups, s_a, bias, bias_dtype, out, out_dtype,
                          ldo, ic_epi{}, stream);
}

int ic_gemv_w4a16(const void* x, int dtype, int64_t M, int64_t K, int64_t ldx, const uint8_t* w_packed, int64_t N,
                  int64_t ldw, const float* s_w, int64_t num_groups, const void* bias, int bias_dtype, void* out,
                  int64_t ldo, void* stream) {
  const char* who = "ic_gemv_w4a16";
  if (dtype != IC_DTYPE_F16 && dtype != IC_DTYPE_BF16)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: activation dtype must be f16/bf16", who);
  int rc = check_gemv_common(who, M, K, N, ldx, ldo, bias, bias_dtype);
  if (rc) return rc;
  if (num_groups < 1 || K % num_groups != 0 || (num_groups > 1 && (K / num_groups) % 32 != 0))
    return ic_set_error(IC_ERR_UNSUPPORTED, "%s: groups must span multiples of 32 values", who);
  if (M == 0) return IC_OK;
  if (!x || !w_packed || !s_w || !out) return ic_set_error(IC_ERR_INVALID_ARG, "%s: null pointer", who);
  if (!ic_gemv_applicable(M, K, x, ldx * 2, w_packed, ldw) || ldw * 2 < K)
    return ic_set_error(IC_ERR_UNSUPPORTED, "%s: operands must be 16-byte aligned", who);
  const int G = (int)num_groups, gsize = (int)(K / num_groups);
  const dim3 grid((unsigned)((N + 15) / 16));
  hipStream_t st = (hipStream_t)stream;
  const int64_t xl_bytes = M * K * 2;
  const bool xl = xl_bytes <= kXlBytes;
  const size_t shm = (size_t)((16 * G + 3) & ~3) * 4 + (xl ? (size_t)xl_bytes : 0);  // at most 48 KB
  auto args = [&](auto kern) {
    kern<<<grid, kGT, shm, st>>>((const u16*)x, ldx, w_packed, ldw, s_w, G, gsize, bias, bias_dtype, (u16*)out, ldo,
                                 (int)M, (int)N, (int)K);
  };
  if (dtype == IC_DTYPE_F16) {
    if (xl) args(gemv_w4a16_kernel<IC_DTYPE_F16, true>);
    else args(gemv_w4a16_kernel<IC_DTYPE_F16, false>);
  } else {
    if (xl) args(gemv_w4a16_kernel<IC_DTYPE_BF16, true>);
    else args(gemv_w4a16_kernel<IC_DTYPE_BF16, false>);
  }
  return ic_check_launch(who);
}

}  // extern "C"
