// W4A16: fp16/bf16 activations x INT4 weights dequantized on the fly (gfx950).
//
// Replaces unpack_int4_to_float16 (triton_int4_unpack.py:25-88) followed by the
// cuBLAS F.linear of _forward_int4_w4a16 (_ops.py:466-481): the dequantized
// weight w[n,k] = RN_dt(q[n,k] * RN_dt(s[n, k/gs])) is produced in the
// global->LDS copy and consumed by v_mfma_f32_32x32x16_{f16,bf16}; it is never
// written to HBM.  For fp16 this is bit-identical to the reference unpack
// (an fp16 product of two fp16 values); the reference rejects bf16 here and
// its PyTorch fallback rounds q*s to the activation type, which is what bf16
// does.  Accumulation is fp32 in the MFMA; the epilogue adds the bias (the
// reference drops it on this path) and rounds to the activation type.
//
// Also provides the standalone unpack kernels (INT4->int8 and INT4->fp16/bf16),
// triton_int4_to_int8_unpack.py:26-81 and triton_int4_unpack.py:25-88.
#include <type_traits>

#include "ic_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kRowBytes = 64;  // 32 fp16 K values per LDS row per stage

// 16-byte chunks XOR-swizzled by (row >> 2): conflict-free ds_read_b128 for
// 32-row MFMA fragments on gfx950.
IC_DEV int lds_off(int row, int chunk) { return row * kRowBytes + ((chunk ^ ((row >> 2) & 3)) << 4); }

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

IC_DEV int nib(uint32_t w, int i) {  // i-th nibble (low nibble first), two's complement
  const int v = (w >> (4 * i)) & 0xf;
  return v >= 8 ? v - 16 : v;
}

// One dequantized weight value RN_dt(q * RN_dt(s)), as f32.
template <int DT> IC_DEV float deq1(int q, float s) {
  if constexpr (DT == IC_DTYPE_F16) return (float)((_Float16)q * (_Float16)s);
  else return bf16_to_f32(f32_to_bf16((float)q * bf16_to_f32(f32_to_bf16(s))));
}
template <int DT> IC_DEV u16 deq1_bits(int q, float s) {
  if constexpr (DT == IC_DTYPE_F16) return __builtin_bit_cast(u16, (_Float16)((_Float16)q * (_Float16)s));
  else return f32_to_bf16((float)q * bf16_to_f32(f32_to_bf16(s)));
}
// Dequantize 8 nibbles of one packed dword to 8 values of type DT (bits).
template <int DT> IC_DEV void deq8(uint32_t P, float s, u16* out) {
#pragma unroll
  for (int i = 0; i < 8; ++i) out[i] = deq1_bits<DT>(nib(P, i), s);
}

template <int BM, int BN, int DT>
__global__ __launch_bounds__(kThreads, 1) void gemm_w4a16_kernel(
    const u16* __restrict__ A, int64_t lda, const uint8_t* __restrict__ B, int64_t ldb,
    const float* __restrict__ s_w, int G, int gsize, const void* __restrict__ bias, int bias_dt,
    u16* __restrict__ C, int64_t ldc, int M, int N, int K) {
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int A_CH = BM * 4 / kThreads;  // 16-byte chunks (8 values) per thread
  constexpr int B_CH = BN / kThreads;      // one packed 16-byte chunk (32 values) per B row
  constexpr int STAGE = (BM + BN) * kRowBytes;
  static_assert(TM >= 1 && TN >= 1 && A_CH >= 1 && B_CH >= 1, "tile too small");
  extern __shared__ __attribute__((aligned(16))) char smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wr = wave >> 1, wc = wave & 1;
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int tm, tn;
  tile_coords(blockIdx.x, tiles_m * tiles_n, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int KT = K / 32;

  v4u ra[A_CH], rb[B_CH];
  float rs[B_CH];
  auto gload = [&](int kt) {
    const int k0 = kt * 32;
#pragma unroll
    for (int c = 0; c < A_CH; ++c) {
      const int q = tid + kThreads * c;
      const int row = min(m0 + (q >> 2), M - 1);
      ra[c] = *(const v4u*)(A + (int64_t)row * lda + k0 + (q & 3) * 8);
    }
#pragma unroll
    for (int c = 0; c < B_CH; ++c) {
      const int row = min(n0 + tid + kThreads * c, N - 1);
      rb[c] = *(const v4u*)(B + (int64_t)row * ldb + (k0 >> 1));
      rs[c] = s_w[(int64_t)row * G + (G > 1 ? k0 / gsize : 0)];
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
      const int row = tid + kThreads * c;
      const uint32_t pw[4] = {rb[c].x, rb[c].y, rb[c].z, rb[c].w};
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        u16 h[8];
        deq8<DT>(pw[d], rs[c], h);
        v4u o;
        o.x = h[0] | ((uint32_t)h[1] << 16);
        o.y = h[2] | ((uint32_t)h[3] << 16);
        o.z = h[4] | ((uint32_t)h[5] << 16);
        o.w = h[6] | ((uint32_t)h[7] << 16);
        *(v4u*)(sB + lds_off(row, d)) = o;
      }
    }
  };

  v16f acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = v16f{};

  auto compute = [&](int buf) {
    const char* sA = smem + buf * STAGE;
    const char* sB = sA + BM * kRowBytes;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int ch = 2 * ks + (lane >> 5);
      v4u a[TM], b[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) a[i] = *(const v4u*)(sA + lds_off(wr * WM + i * 32 + (lane & 31), ch));
#pragma unroll
      for (int j = 0; j < TN; ++j) b[j] = *(const v4u*)(sB + lds_off(wc * WN + j * 32 + (lane & 31), ch));
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          if constexpr (DT == IC_DTYPE_F16)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, a[i]),
                                                               __builtin_bit_cast(v8h, b[j]), acc[i][j], 0, 0, 0);
          else
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a[i]),
                                                                __builtin_bit_cast(v8bf, b[j]), acc[i][j], 0, 0, 0);
        }
    }
  };

  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    if (kt + 1 < KT) gload(kt + 1);
    compute(kt & 1);
    if (kt + 1 < KT) sstore((kt + 1) & 1);
    __syncthreads();
  }

#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int n = n0 + wc * WN + j * 32 + (lane & 31);
    const float b = bias != nullptr ? ld_any_f32(bias, bias_dt, min(n, N - 1)) : 0.0f;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wr * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m >= M || n >= N) continue;
        float v = acc[i][j][r];
        if (bias != nullptr) v = v + b;
        st_from_f32<DT>(C, (int64_t)m * ldc + n, v);
      }
  }
}

// Shape-generic fallback: one thread per output, fp32 dot product.
template <int DT>
__global__ __launch_bounds__(256) void gemm_w4a16_generic_kernel(
    const u16* __restrict__ A, int64_t lda, const uint8_t* __restrict__ B, int64_t ldb,
    const float* __restrict__ s_w, int G, int gsize, const void* __restrict__ bias, int bias_dt,
    u16* __restrict__ C, int64_t ldc, int M, int N, int K) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  const int m = blockIdx.y;
  if (n >= N || m >= M) return;
  float acc = 0.0f;
  for (int k = 0; k < K; ++k) {
    const int q = nib((uint32_t)B[(int64_t)n * ldb + (k >> 1)], k & 1);
    const float w = deq1<DT>(q, s_w[(int64_t)n * G + (G > 1 ? k / gsize : 0)]);
    acc = __builtin_fmaf(ld_as_f32<DT>(A, (int64_t)m * lda + k), w, acc);
  }
  if (bias != nullptr) acc = acc + ld_any_f32(bias, bias_dt, n);
  st_from_f32<DT>(C, (int64_t)m * ldc + n, acc);
}

template <int BM, int BN, int DT>
hipError_t launch_w4a16(const u16* A, int64_t lda, const uint8_t* B, int64_t ldb, const float* s_w,
                        int G, int gsize, const void* bias, int bias_dt, u16* C, int64_t ldc, int M,
                        int N, int K, hipStream_t st) {
  const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  const size_t shm = 2 * (BM + BN) * kRowBytes;
  gemm_w4a16_kernel<BM, BN, DT><<<dim3(tiles), dim3(kThreads), shm, st>>>(A, lda, B, ldb, s_w, G, gsize,
                                                                          bias, bias_dt, C, ldc, M, N, K);
  return hipGetLastError();
}

template <int DT>
hipError_t run_w4a16(const u16* A, int64_t lda, const uint8_t* B, int64_t ldb, const float* s_w, int G,
                     int gsize, const void* bias, int bias_dt, u16* C, int64_t ldc, int M, int N, int K,
                     bool mfma_ok, hipStream_t st) {
  if (mfma_ok) {
    if (M >= 256 && N >= 256) return launch_w4a16<256, 256, DT>(A, lda, B, ldb, s_w, G, gsize, bias, bias_dt, C, ldc, M, N, K, st);
    return launch_w4a16<128, 256, DT>(A, lda, B, ldb, s_w, G, gsize, bias, bias_dt, C, ldc, M, N, K, st);
  }
  dim3 grid((unsigned)((N + 255) / 256), (unsigned)M);
  gemm_w4a16_generic_kernel<DT><<<grid, dim3(256), 0, st>>>(A, lda, B, ldb, s_w, G, gsize, bias, bias_dt, C, ldc, M, N, K);
  return hipGetLastError();
}

__global__ void unpack_i8_kernel(const uint8_t* __restrict__ P, int64_t ldp, int8_t* __restrict__ O,
                                 int64_t ldo, int N, int K) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)N * K;
  if (idx >= total) return;
  const int n = (int)(idx / K), k = (int)(idx % K);
  const int v = (P[(int64_t)n * ldp + (k >> 1)] >> (4 * (k & 1))) & 0xf;
  O[(int64_t)n * ldo + k] = (int8_t)(v >= 8 ? v - 16 : v);
}

template <int DT>
__global__ void unpack_fp_kernel(const uint8_t* __restrict__ P, int64_t ldp, const float* __restrict__ s_w,
                                 int G, int gsize, u16* __restrict__ O, int64_t ldo, int N, int K) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)N * K;
  if (idx >= total) return;
  const int n = (int)(idx / K), k = (int)(idx % K);
  const int q = nib((uint32_t)P[(int64_t)n * ldp + (k >> 1)], k & 1);
  O[(int64_t)n * ldo + k] = deq1_bits<DT>(q, s_w[(int64_t)n * G + (G > 1 ? k / gsize : 0)]);
}

}  // namespace

extern "C" {

int ic_gemm_w4a16(const void* x, int dtype, int64_t M, int64_t K, int64_t ldx, const uint8_t* w_packed,
                  int64_t N, int64_t ldw, const float* s_w, int64_t num_groups, const void* bias,
                  int bias_dtype, void* out, int64_t ldo, void* stream) {
  const char* who = "ic_gemm_w4a16";
  if (dtype != IC_DTYPE_F16 && dtype != IC_DTYPE_BF16)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: activation dtype must be f16/bf16", who);
  if (M < 0 || N <= 0 || K <= 0 || ldx < K || ldo < N || ldw * 2 < K || num_groups < 1 ||
      K % num_groups != 0)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: bad shape M=%lld N=%lld K=%lld groups=%lld", who,
                        (long long)M, (long long)N, (long long)K, (long long)num_groups);
  if (bias && bias_dtype != IC_DTYPE_F16 && bias_dtype != IC_DTYPE_BF16 && bias_dtype != IC_DTYPE_F32)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: bias dtype must be f16/bf16/f32", who);
  if (M == 0) return IC_OK;
  if (!x || !w_packed || !s_w || !out) return ic_set_error(IC_ERR_INVALID_ARG, "%s: null pointer", who);
  if (ic_gemv_applicable(M, K, x, ldx * 2, w_packed, ldw) && (num_groups == 1 || (K / num_groups) % 32 == 0))
    return ic_gemv_w4a16(x, dtype, M, K, ldx, w_packed, N, ldw, s_w, num_groups, bias, bias_dtype, out, ldo, stream);
  const int G = (int)num_groups, gsize = (int)(K / num_groups);
  const bool mfma_ok = (K % 32 == 0) && (G == 1 || gsize % 32 == 0) && !((uintptr_t)x & 15) &&
                       !((uintptr_t)w_packed & 15) && !((ldx * 2) & 15) && !(ldw & 15);
  hipStream_t st = (hipStream_t)stream;
  hipError_t e = dtype == IC_DTYPE_F16
                     ? run_w4a16<IC_DTYPE_F16>((const u16*)x, ldx, w_packed, ldw, s_w, G, gsize, bias, bias_dtype,
                                               (u16*)out, ldo, (int)M, (int)N, (int)K, mfma_ok, st)
                     : run_w4a16<IC_DTYPE_BF16>((const u16*)x, ldx, w_packed, ldw, s_w, G, gsize, bias, bias_dtype,
                                                (u16*)out, ldo, (int)M, (int)N, (int)K, mfma_ok, st);
  if (e != hipSuccess) return ic_set_error(IC_ERR_LAUNCH, "%s: %s", who, hipGetErrorString(e));
  return IC_OK;
}

int ic_unpack_int4_to_int8(const uint8_t* packed, int64_t N, int64_t K, int64_t ldp, int8_t* out,
                           int64_t ldo, void* stream) {
  if (N < 0 || K < 0 || ldp * 2 < K || ldo < K || (N * K > 0 && (!packed || !out)))
    return ic_set_error(IC_ERR_INVALID_ARG, "ic_unpack_int4_to_int8: bad arguments");
  const int64_t total = N * K;
  if (total == 0) return IC_OK;
  unpack_i8_kernel<<<dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream>>>(
      packed, ldp, out, ldo, (int)N, (int)K);
  return ic_check_launch("ic_unpack_int4_to_int8");
}

int ic_unpack_int4_to_float(const uint8_t* packed, const float* s_w, int64_t num_groups, int64_t N,
                            int64_t K, int64_t ldp, void* out, int out_dtype, int64_t ldo, void* stream) {
  if (N < 0 || K < 0 || ldp * 2 < K || ldo < K || num_groups < 1 || (K > 0 && K % num_groups != 0) ||
      (N * K > 0 && (!packed || !out || !s_w)))
    return ic_set_error(IC_ERR_INVALID_ARG, "ic_unpack_int4_to_float: bad arguments");
  if (out_dtype != IC_DTYPE_F16 && out_dtype != IC_DTYPE_BF16)
    return ic_set_error(IC_ERR_INVALID_ARG, "ic_unpack_int4_to_float: out dtype must be f16/bf16");
  const int64_t total = N * K;
  if (total == 0) return IC_OK;
  const int G = (int)num_groups, gsize = (int)(K / num_groups);
  dim3 grid((unsigned)((total + 255) / 256));
  if (out_dtype == IC_DTYPE_F16)
    unpack_fp_kernel<IC_DTYPE_F16><<<grid, dim3(256), 0, (hipStream_t)stream>>>(packed, ldp, s_w, G, gsize, (u16*)out, ldo, (int)N, (int)K);
  else
    unpack_fp_kernel<IC_DTYPE_BF16><<<grid, dim3(256), 0, (hipStream_t)stream>>>(packed, ldp, s_w, G, gsize, (u16*)out, ldo, (int)N, (int)K);
  return ic_check_launch("ic_unpack_int4_to_float");
}

}  // extern "C"
