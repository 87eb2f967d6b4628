// Row normalisation fused with per-token INT8 quantization (gfx950):
// LayerNorm, RMSNorm or softmax over each row, then the dynamic quantization
// of the normalised row, in one kernel.  Replaces fused_layernorm_quantize
// (kernels/triton_quantize.py:209-345), fused_rmsnorm_quantize (:348-459) and
// fused_softmax_quantize (:462-567).
//
// Arithmetic (per row of K values x, read as f32):
//   LayerNorm  mean = RN32(S1 / K), var = max(S2 / K - (S1 / K)^2, 0) with
//              S1 = sum x, S2 = sum x^2 in fp64; rstd = RN32(1 / sqrt(var + eps));
//              y = RN32(RN32(x - mean) * rstd) * gamma (+ beta), each step RN32
//   RMSNorm    rstd = RN32(1 / sqrt(sum x^2 / K + eps)) with the sum in fp64;
//              y = RN32(x * rstd) * gamma
//   softmax    m = max x; e = exp(RN32(x - m)) (f32 expf); inv = RN32(1 / sum e), sum in fp64;
//              y = RN32(e * inv)
// then s = max(max|y|, 1e-8) / 127 and q = trunc(RN32(y / s) +- 0.5) clamped to
// [-128, 127], the reference GPU quantization rule (triton_quantize.py:266-274).
// The reference accumulates its statistics in f32 in Triton's reduction order;
// the fp64 sums here are order-independent to well below f32 resolution, and the
// reference tests bound the codes to +-1 of an f32 PyTorch reference.
//
// One 256-thread workgroup per row, persistent over rows.  Rows with K % 8 == 0,
// K <= 16384 and 16-byte aligned rows are held in registers (8 contiguous values
// per thread and chunk, up to 8 chunks); other rows take a generic kernel that
// re-reads the row from global memory in each pass.
#include "ic_common.h"

namespace {

constexpr int kNQThreads = 256;
constexpr int kNQMaxChunks = 8;  // 8 values each: K <= 16384 in registers

IC_DEV double block_sum(double v, double* red) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  __syncthreads();  // red is free (previous reduction consumed)
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  double t = red[0];
#pragma unroll
  for (int w = 1; w < kNQThreads / 64; ++w) t += red[w];
  return t;
}

IC_DEV float block_max(float v, float* red) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = __builtin_fmaxf(v, __shfl_xor(v, o, 64));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = red[0];
#pragma unroll
  for (int w = 1; w < kNQThreads / 64; ++w) t = __builtin_fmaxf(t, red[w]);
  return t;
}

// Statistics of one row for KIND, from a per-thread visitor over its values:
// fills a (mean or max) and b (rstd or 1/sum) used by finish().
template <int KIND>
struct RowStats {
  float a = 0.0f, b = 0.0f;
};

template <int KIND>
IC_DEV float finish(float x, const RowStats<KIND>& st, float g, float be, bool has_beta) {
  if constexpr (KIND == IC_NORM_LAYER) {
    float y = (x - st.a) * st.b;
    y = y * g;
    if (has_beta) y = y + be;
    return y;
  } else if constexpr (KIND == IC_NORM_RMS) {
    return (x * st.b) * g;
  } else {
    return expf(x - st.a) * st.b;
  }
}

template <int DT>
IC_DEV void load8(const void* row, int c, float* v) {
  if constexpr (DT == IC_DTYPE_F32) {
    const v4f a = ((const v4f*)row)[2 * c], b = ((const v4f*)row)[2 * c + 1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    const v4u p = ((const v4u*)row)[c];
    const uint32_t w[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (DT == IC_DTYPE_F16) {
        v[2 * i] = f16_to_f32((u16)(w[i] & 0xffffu));
        v[2 * i + 1] = f16_to_f32((u16)(w[i] >> 16));
      } else {
        v[2 * i] = bf16_to_f32((u16)(w[i] & 0xffffu));
        v[2 * i + 1] = bf16_to_f32((u16)(w[i] >> 16));
      }
    }
  }
}

// Register-resident rows: chunk c = tid + 256 * i holds values 8c .. 8c + 7.
template <int DT, int KIND, int NC>
__global__ __launch_bounds__(kNQThreads) void norm_quant_kernel(
    const void* __restrict__ x, int64_t ldx, int M, int K, const float* __restrict__ gamma,
    const float* __restrict__ beta, float eps, int8_t* __restrict__ q_out, int64_t ldq,
    float* __restrict__ s_out) {
  __shared__ double red_d[kNQThreads / 64];
  __shared__ float red_f[kNQThreads / 64];
  const int tid = threadIdx.x;
  const int nchunks = K / 8;
  const int esz = DT == IC_DTYPE_F32 ? 4 : 2;
  for (int row = blockIdx.x; row < M; row += gridDim.x) {
    const char* xr = (const char*)x + (int64_t)row * ldx * esz;
    float v[NC][8];
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = tid + kNQThreads * i;
      if (c < nchunks) load8<DT>(xr, c, v[i]);
      else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[i][e] = 0.0f;
      }
    }
    RowStats<KIND> st;
    if constexpr (KIND == IC_NORM_LAYER) {
      double s1 = 0.0, s2 = 0.0;
#pragma unroll
      for (int i = 0; i < NC; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          s1 += (double)v[i][e];
          s2 += (double)v[i][e] * (double)v[i][e];
        }
      const double mean = block_sum(s1, red_d) / K;
      const double var = __builtin_fmax(block_sum(s2, red_d) / K - mean * mean, 0.0);
      st.a = (float)mean;
      st.b = (float)(1.0 / __builtin_sqrt(var + (double)eps));
    } else if constexpr (KIND == IC_NORM_RMS) {
      double s2 = 0.0;
#pragma unroll
      for (int i = 0; i < NC; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) s2 += (double)v[i][e] * (double)v[i][e];
      st.b = (float)(1.0 / __builtin_sqrt(block_sum(s2, red_d) / K + (double)eps));
    } else {
      float m = -__builtin_huge_valf();
#pragma unroll
      for (int i = 0; i < NC; ++i) {
        if (tid + kNQThreads * i >= nchunks) break;
#pragma unroll
        for (int e = 0; e < 8; ++e) m = __builtin_fmaxf(m, v[i][e]);
      }
      st.a = block_max(m, red_f);
      double se = 0.0;
#pragma unroll
      for (int i = 0; i < NC; ++i) {
        if (tid + kNQThreads * i >= nchunks) break;
#pragma unroll
        for (int e = 0; e < 8; ++e) se += (double)expf(v[i][e] - st.a);
      }
      st.b = (float)(1.0 / block_sum(se, red_d));
    }
    // abs-max of the normalised row
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = tid + kNQThreads * i;
      if (c >= nchunks) break;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int k = 8 * c + e;
        const float g = KIND == IC_SOFTMAX ? 1.0f : gamma[k];
        const float be = beta != nullptr ? beta[k] : 0.0f;
        amax = __builtin_fmaxf(amax, __builtin_fabsf(finish<KIND>(v[i][e], st, g, be, beta != nullptr)));
      }
    }
    const float s = quant_scale(block_max(amax, red_f));
    const double rs = 1.0 / (double)s;
    if (tid == 0) s_out[row] = s;
    int8_t* qr = q_out + (int64_t)row * ldq;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = tid + kNQThreads * i;
      if (c >= nchunks) break;
      int code[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int k = 8 * c + e;
        const float g = KIND == IC_SOFTMAX ? 1.0f : gamma[k];
        const float be = beta != nullptr ? beta[k] : 0.0f;
        code[e] = quant_code(finish<KIND>(v[i][e], st, g, be, beta != nullptr), rs);
      }
      ((uint2*)qr)[c] = uint2{pack4_lo_bytes(code[0], code[1], code[2], code[3]),
                              pack4_lo_bytes(code[4], code[5], code[6], code[7])};
    }
  }
}

// Any K and alignment: every pass re-reads the row (L2-resident for the rows
// this path sees).
template <int DT, int KIND>
__global__ __launch_bounds__(kNQThreads) void norm_quant_generic_kernel(
    const void* __restrict__ x, int64_t ldx, int M, int K, const float* __restrict__ gamma,
    const float* __restrict__ beta, float eps, int8_t* __restrict__ q_out, int64_t ldq,
    float* __restrict__ s_out) {
  __shared__ double red_d[kNQThreads / 64];
  __shared__ float red_f[kNQThreads / 64];
  const int tid = threadIdx.x;
  for (int row = blockIdx.x; row < M; row += gridDim.x) {
    const void* xr = (const char*)x + (int64_t)row * ldx * (DT == IC_DTYPE_F32 ? 4 : 2);
    RowStats<KIND> st;
    if constexpr (KIND == IC_NORM_LAYER) {
      double s1 = 0.0, s2 = 0.0;
      for (int k = tid; k < K; k += kNQThreads) {
        const double d = (double)ld_as_f32<DT>(xr, k);
        s1 += d;
        s2 += d * d;
      }
      const double mean = block_sum(s1, red_d) / K;
      const double var = __builtin_fmax(block_sum(s2, red_d) / K - mean * mean, 0.0);
      st.a = (float)mean;
      st.b = (float)(1.0 / __builtin_sqrt(var + (double)eps));
    } else if constexpr (KIND == IC_NORM_RMS) {
      double s2 = 0.0;
      for (int k = tid; k < K; k += kNQThreads) {
        const double d = (double)ld_as_f32<DT>(xr, k);
        s2 += d * d;
      }
      st.b = (float)(1.0 / __builtin_sqrt(block_sum(s2, red_d) / K + (double)eps));
    } else {
      float m = -__builtin_huge_valf();
      for (int k = tid; k < K; k += kNQThreads) m = __builtin_fmaxf(m, ld_as_f32<DT>(xr, k));
      st.a = block_max(m, red_f);
      double se = 0.0;
      for (int k = tid; k < K; k += kNQThreads) se += (double)expf(ld_as_f32<DT>(xr, k) - st.a);
      st.b = (float)(1.0 / block_sum(se, red_d));
    }
    float amax = 0.0f;
    for (int k = tid; k < K; k += kNQThreads) {
      const float g = KIND == IC_SOFTMAX ? 1.0f : gamma[k];
      const float be = beta != nullptr ? beta[k] : 0.0f;
      amax = __builtin_fmaxf(amax, __builtin_fabsf(finish<KIND>(ld_as_f32<DT>(xr, k), st, g, be, beta != nullptr)));
    }
    const float s = quant_scale(block_max(amax, red_f));
    const double rs = 1.0 / (double)s;
    if (tid == 0) s_out[row] = s;
    for (int k = tid; k < K; k += kNQThreads) {
      const float g = KIND == IC_SOFTMAX ? 1.0f : gamma[k];
      const float be = beta != nullptr ? beta[k] : 0.0f;
      q_out[(int64_t)row * ldq + k] = (int8_t)quant_code(finish<KIND>(ld_as_f32<DT>(xr, k), st, g, be, beta != nullptr), rs);
    }
  }
}

template <int DT, int KIND>
hipError_t launch_nq(const void* x, int64_t ldx, int M, int K, const float* g, const float* b, float eps,
                     int8_t* q, int64_t ldq, float* s, hipStream_t st) {
  const int grid = (int)std::min<int64_t>(M, (int64_t)ic_num_cus() * 8);
  const bool vec = K % 8 == 0 && K <= kNQMaxChunks * 8 * kNQThreads && ((uintptr_t)x & 15) == 0 &&
                   (ldx * (DT == IC_DTYPE_F32 ? 4 : 2)) % 16 == 0 && ((uintptr_t)q & 7) == 0 && ldq % 8 == 0;
  if (vec) {
    const int nc = (K / 8 + kNQThreads - 1) / kNQThreads;
    if (nc <= 1) norm_quant_kernel<DT, KIND, 1><<<grid, kNQThreads, 0, st>>>(x, ldx, M, K, g, b, eps, q, ldq, s);
    else if (nc <= 2) norm_quant_kernel<DT, KIND, 2><<<grid, kNQThreads, 0, st>>>(x, ldx, M, K, g, b, eps, q, ldq, s);
    else if (nc <= 4) norm_quant_kernel<DT, KIND, 4><<<grid, kNQThreads, 0, st>>>(x, ldx, M, K, g, b, eps, q, ldq, s);
    else norm_quant_kernel<DT, KIND, 8><<<grid, kNQThreads, 0, st>>>(x, ldx, M, K, g, b, eps, q, ldq, s);
  } else {
    norm_quant_generic_kernel<DT, KIND><<<grid, kNQThreads, 0, st>>>(x, ldx, M, K, g, b, eps, q, ldq, s);
  }
  return hipGetLastError();
}

template <int DT>
hipError_t launch_nq_kind(int kind, const void* x, int64_t ldx, int M, int K, const float* g, const float* b,
                          float eps, int8_t* q, int64_t ldq, float* s, hipStream_t st) {
  switch (kind) {
    case IC_NORM_LAYER: return launch_nq<DT, IC_NORM_LAYER>(x, ldx, M, K, g, b, eps, q, ldq, s, st);
    case IC_NORM_RMS: return launch_nq<DT, IC_NORM_RMS>(x, ldx, M, K, g, b, eps, q, ldq, s, st);
    default: return launch_nq<DT, IC_SOFTMAX>(x, ldx, M, K, g, b, eps, q, ldq, s, st);
  }
}

}  // namespace

extern "C" int ic_norm_quantize(const void* x, int dtype, int64_t M, int64_t K, int64_t ldx, int kind,
                                const float* gamma, const float* beta, float eps, int8_t* q_out, int64_t ldq,
                                float* s_out, void* stream) {
  if (kind != IC_NORM_LAYER && kind != IC_NORM_RMS && kind != IC_SOFTMAX)
    return ic_set_error(IC_ERR_INVALID_ARG, "ic_norm_quantize: kind must be IC_NORM_LAYER, IC_NORM_RMS or IC_SOFTMAX");
  if (dtype != IC_DTYPE_F16 && dtype != IC_DTYPE_BF16 && dtype != IC_DTYPE_F32)
    return ic_set_error(IC_ERR_INVALID_ARG, "ic_norm_quantize: dtype must be f16/bf16/f32");
  if (M < 0 || K <= 0 || ldx < K || ldq < K || M > INT32_MAX || K > INT32_MAX)
    return ic_set_error(IC_ERR_INVALID_ARG, "ic_norm_quantize: bad shape M=%lld K=%lld ldx=%lld ldq=%lld",
                        (long long)M, (long long)K, (long long)ldx, (long long)ldq);
  if (kind == IC_SOFTMAX && (gamma != nullptr || beta != nullptr))
    return ic_set_error(IC_ERR_INVALID_ARG, "ic_norm_quantize: softmax takes no gamma/beta");
  if (kind != IC_SOFTMAX && gamma == nullptr)
    return ic_set_error(IC_ERR_INVALID_ARG, "ic_norm_quantize: LayerNorm/RMSNorm need gamma");
  if (kind == IC_NORM_RMS && beta != nullptr)
    return ic_set_error(IC_ERR_INVALID_ARG, "ic_norm_quantize: RMSNorm takes no beta");
  if (!(eps >= 0.0f)) return ic_set_error(IC_ERR_INVALID_ARG, "ic_norm_quantize: eps must be >= 0");
  if (M == 0) return IC_OK;
  if (x == nullptr || q_out == nullptr || s_out == nullptr)
    return ic_set_error(IC_ERR_INVALID_ARG, "ic_norm_quantize: null pointer argument");
  hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  switch (dtype) {
    case IC_DTYPE_F16: e = launch_nq_kind<IC_DTYPE_F16>(kind, x, ldx, (int)M, (int)K, gamma, beta, eps, q_out, ldq, s_out, st); break;
    case IC_DTYPE_BF16: e = launch_nq_kind<IC_DTYPE_BF16>(kind, x, ldx, (int)M, (int)K, gamma, beta, eps, q_out, ldq, s_out, st); break;
    default: e = launch_nq_kind<IC_DTYPE_F32>(kind, x, ldx, (int)M, (int)K, gamma, beta, eps, q_out, ldq, s_out, st); break;
  }
  if (e != hipSuccess) return ic_set_error(IC_ERR_LAUNCH, "ic_norm_quantize: %s", hipGetErrorString(e));
  return IC_OK;
}
