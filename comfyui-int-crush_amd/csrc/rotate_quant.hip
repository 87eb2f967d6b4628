// Fused activation preparation + per-token dynamic INT8 quantization (gfx950).
//
// One workgroup (256 threads, 4 waves) owns one activation row.  The row is
// read from HBM once and the INT8 codes are written once; every intermediate
// lives in registers or LDS:
//
//   x[K_in] (fp16/bf16/f32)
//     -> SmoothRot divide, rounded to the activation type      (_ops.py:347-350)
//     -> zero pad to a multiple of R, block Hadamard of size R   (_quant_utils.py:117-147)
//        computed with fp64 butterflies: exact for fp16 inputs, then rounded
//        once to the activation type
//     -> zero pad to K_w                                          (_ops.py:355-358)
//     -> PermuQuant gather out[j] = rot[perm[j]]                  (_ops.py:360-363)
//     -> optional old-SmoothQuant divide after the gather         (_ops.py:529-533)
//     -> per-row abs-max, s = max(m,1e-8)/127, q = trunc(v/s +- 0.5) (triton_quantize.py:109-146)
//
// The Hadamard H_R = (H4/2)^{(x)k}, R = 4^k, acts on each base-4 digit of the
// in-block index with the radix-4 butterfly y_i = s/2 - x_{3-i}, s = sum(x).
// A tile of 4096 positions is spread as 16 contiguous elements per thread
// (digits 0-1 in registers); digits 2-3 are reached through one LDS transpose
// among 16 threads, digits 4-5 through a second transpose among 256 threads.
#include "rq_row.h"

namespace {

using namespace rq;

// LOG4R: 0 = no rotation, 2..6 = rot size 16..4096.  QUANT: write INT8 codes and
// scales; otherwise write the prepared activation in the input type.
template <int DT, int LOG4R, bool QUANT>
__global__ __launch_bounds__(kThreads) void rotate_quant_kernel(
    const void* __restrict__ x, int64_t ldx, int K_in,
    const float* __restrict__ sr_rcp, const float* __restrict__ sr_f,
    int K_w, const int32_t* __restrict__ perm,
    const float* __restrict__ sm_rcp, const float* __restrict__ sm_f,
    int8_t* __restrict__ q_out, int64_t ldq, float* __restrict__ s_out,
    void* __restrict__ y_out, int64_t ldy) {
  constexpr int R = LOG4R == 0 ? 1 : (1 << (2 * LOG4R));
  constexpr int ESZ = DT == IC_DTYPE_F32 ? 4 : 2;

  __shared__ double tbuf[kTbufDoubles];  // 36 KB; reused as the row buffer
  __shared__ float red[kThreads / 64];
  __shared__ uint32_t xred[DT == IC_DTYPE_BF16 && LOG4R == 6 ? kXredWords : 1];

  const int t = threadIdx.x;
  const int64_t row = blockIdx.x;
  const char* xrow = (const char*)x + row * ldx * ESZ;
  const int K_r = LOG4R == 0 ? K_in : ((K_in + R - 1) / R) * R;  // rotated width
  const bool xvec = ((((uintptr_t)xrow) & 15) == 0);
  const bool fvec = (sr_rcp == nullptr || (((uintptr_t)sr_rcp) & 15) == 0) &&
                    (sm_rcp == nullptr || (((uintptr_t)sm_rcp) & 15) == 0);
  const int ntiles = (K_w + kTile - 1) / kTile;

  // Rotated, rounded values of this thread (exact values of type DT) per tile.
  float val[kMaxTiles][16];
#pragma unroll
  for (int tile = 0; tile < kMaxTiles; ++tile) {
    if (tile >= ntiles) break;
    // load + SmoothRot divide (16 contiguous positions per thread)
    const int p0 = tile * kTile + 16 * t;
    float xs[16];
    load16<DT>(xrow, p0, K_in, xvec, xs);
    if (sr_rcp != nullptr) {
      float rc[16];
      load16<IC_DTYPE_F32>(sr_rcp, p0, K_in, fvec, rc);
      smoothrot_divide16<DT>(xs, rc, sr_f, p0, K_in);
    }
    rotate_tile<DT, LOG4R>(xs, tbuf, xred, tile * kTile, K_r, val[tile]);
  }
  char* rowbuf = (char*)tbuf;
  publish_row<DT, LOG4R, kMaxTiles>(val, ntiles, K_w, rowbuf);

  // gather (perm), old-smooth divide, abs-max.  Thread t owns output
  // positions o = 16*(t + 256*c) + j.
  float m = 0.0f;
#pragma unroll
  for (int c = 0; c < kMaxTiles; ++c) {
    if (c >= ntiles) break;
    const int o0 = 16 * (t + kThreads * c);
    int src[16];
    if (perm != nullptr) {
      load16i(perm, o0, K_w, src);
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) src[j] = o0 + j;
    }
    float smr[16];
    if (sm_rcp != nullptr) load16<IC_DTYPE_F32>(sm_rcp, o0, K_w, fvec, smr);
    m = gather16<DT>(rowbuf, src, sm_rcp != nullptr, smr, sm_f, o0, K_w, val[c], m);
  }

  if constexpr (!QUANT) {
#pragma unroll
    for (int c = 0; c < kMaxTiles; ++c) {
      if (c >= ntiles) break;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int o = 16 * (t + kThreads * c) + j;
        if (o < K_w) st_from_f32<DT>((char*)y_out + row * ldy * ESZ, o, val[c][j]);
      }
    }
  } else {
    const float s = row_scale(m, red);
    const double rs = 1.0 / (double)s;
    if (t == 0) s_out[row] = s;
    int8_t* qrow = q_out + row * ldq;
#pragma unroll
    for (int c = 0; c < kMaxTiles; ++c) {
      if (c >= ntiles) break;
      const int o0 = 16 * (t + kThreads * c);
      if (o0 >= K_w) break;
      store_codes16(val[c], rs, qrow, o0, K_w);
    }
  }
}

// Row-streaming two-pass quantizer for rows wider than the fused kernel holds
// (dynamic_quantize_activation semantics, triton_quantize.py:109-146).
template <int DT>
__global__ __launch_bounds__(kThreads) void quant_rows_kernel(
    const void* __restrict__ x, int64_t ldx, int K, int8_t* __restrict__ q_out, int64_t ldq,
    float* __restrict__ s_out) {
  constexpr int ESZ = DT == IC_DTYPE_F32 ? 4 : 2;
  __shared__ float red[kThreads / 64];
  const int t = threadIdx.x;
  const int64_t row = blockIdx.x;
  const char* xrow = (const char*)x + row * ldx * ESZ;
  float m = 0.0f;
  for (int k = t; k < K; k += kThreads) m = __builtin_fmaxf(m, __builtin_fabsf(ld_as_f32<DT>(xrow, k)));
  m = wave_max(m);
  if ((t & 63) == 0) red[t >> 6] = m;
  __syncthreads();
  m = __builtin_fmaxf(__builtin_fmaxf(red[0], red[1]), __builtin_fmaxf(red[2], red[3]));
  const float s = quant_scale(m);
  const double rs = 1.0 / (double)s;
  if (t == 0) s_out[row] = s;
  for (int k = t; k < K; k += kThreads) q_out[row * ldq + k] = (int8_t)quant_code(ld_as_f32<DT>(xrow, k), rs);
}

// Second pass of the preparation for rows wider than the fused kernels hold:
// the rotated rows y [M, K_y] (SmoothRot divide and block Hadamard already
// applied, in column chunks) are padded with zeros to K_w, gathered by the
// PermuQuant indices, divided by the old SmoothQuant factors, then quantized
// per token (QUANT) or written in the activation type.  One workgroup per
// row; the quantizing form reads the row twice (abs-max, then codes), the
// second time from L2.
template <int DT, bool QUANT>
__global__ __launch_bounds__(kThreads) void permute_rows_kernel(
    const void* __restrict__ y, int64_t ldy, int K_y, int K_w, const int32_t* __restrict__ perm,
    const float* __restrict__ sm_rcp, const float* __restrict__ sm_f, int8_t* __restrict__ q_out, int64_t ldq,
    float* __restrict__ s_out, void* __restrict__ out, int64_t ldo) {
  constexpr int ESZ = DT == IC_DTYPE_F32 ? 4 : 2;
  __shared__ float red[kThreads / 64];
  const int t = threadIdx.x;
  const int64_t row = blockIdx.x;
  const char* yrow = (const char*)y + row * ldy * ESZ;
  auto value = [&](int o) {
    int src = o;
    if (perm != nullptr) src = (unsigned)perm[o] < (unsigned)K_w ? perm[o] : 0;  // malformed -> position 0
    float v = src < K_y ? ld_as_f32<DT>(yrow, src) : 0.0f;
    if (sm_rcp != nullptr) v = div_round_dt<DT>(v, sm_rcp[o], sm_f, o);
    return v;
  };
  if constexpr (!QUANT) {
    for (int o = t; o < K_w; o += kThreads) st_from_f32<DT>((char*)out + row * ldo * ESZ, o, value(o));
  } else {
    float m = 0.0f;
    for (int o = t; o < K_w; o += kThreads) m = __builtin_fmaxf(m, __builtin_fabsf(value(o)));
    m = wave_max(m);
    if ((t & 63) == 0) red[t >> 6] = m;
    __syncthreads();
    m = __builtin_fmaxf(__builtin_fmaxf(red[0], red[1]), __builtin_fmaxf(red[2], red[3]));
    const float s = quant_scale(m);
    const double rs = 1.0 / (double)s;
    if (t == 0) s_out[row] = s;
    for (int o = t; o < K_w; o += kThreads) q_out[row * ldq + o] = (int8_t)quant_code(value(o), rs);
  }
}

template <int DT>
hipError_t launch_permute_rows(const void* y, int64_t ldy, int64_t M, int64_t K_y, int64_t K_w, const int32_t* perm,
                               const float* sm_rcp, const float* sm_f, int8_t* q_out, int64_t ldq, float* s_out,
                               void* out, int64_t ldo, hipStream_t st) {
  const dim3 grid((unsigned)M), block(kThreads);
  if (q_out != nullptr)
    permute_rows_kernel<DT, true><<<grid, block, 0, st>>>(y, ldy, (int)K_y, (int)K_w, perm, sm_rcp, sm_f, q_out, ldq,
                                                          s_out, nullptr, 0);
  else
    permute_rows_kernel<DT, false><<<grid, block, 0, st>>>(y, ldy, (int)K_y, (int)K_w, perm, sm_rcp, sm_f, nullptr,
                                                           0, nullptr, out, ldo);
  return hipGetLastError();
}

// SmoothRot / SmoothQuant factor preparation: fdt[k] = RN_dt(f[k]) as f32 and
// rcp[k] = RN32(1 / fdt[k]) (IEEE divide).
template <int DT>
__global__ void factor_prep_kernel(const float* __restrict__ f, int K, float* __restrict__ fdt,
                                   float* __restrict__ rcp) {
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= K) return;
  const float v = round_to_dt<DT>(f[k]);
  fdt[k] = v;
  rcp[k] = 1.0f / v;
}

bool fast_path_ok(const ic_rotq_args& a) {
  auto al16 = [](const void* p) { return (((uintptr_t)p) & 15) == 0; };
  if (a.dtype != IC_DTYPE_F16 && a.dtype != IC_DTYPE_BF16) return false;
  if (a.sm_rcp != nullptr || a.q_out == nullptr) return false;
  if (a.K_in % 16 || a.K_w % 16 || a.K_w > (int64_t)kFastMaxTiles * kTile) return false;
  if (a.ldx % 8 || a.ldq % 16 || !al16(a.x) || !al16(a.q_out)) return false;
  if ((a.sr_rcp && !al16(a.sr_rcp)) || (a.perm && !al16(a.perm))) return false;
  return true;
}

template <int DT, int LOG4R, bool QUANT>
hipError_t launch_rq(const ic_rotq_args& a, hipStream_t st) {
  rotate_quant_kernel<DT, LOG4R, QUANT><<<dim3((unsigned)a.M), dim3(kThreads), 0, st>>>(
      a.x, a.ldx, (int)a.K_in, a.sr_rcp, a.sr_f, (int)a.K_w, a.perm, a.sm_rcp, a.sm_f, a.q_out,
      a.ldq, a.s_out, a.y_out, a.ldy);
  return hipGetLastError();
}

template <int DT, bool QUANT>
hipError_t dispatch_rot(const ic_rotq_args& a, hipStream_t st) {
  switch (a.rot_size) {
    case 0: return launch_rq<DT, 0, QUANT>(a, st);
    case 16: return launch_rq<DT, 2, QUANT>(a, st);
    case 64: return launch_rq<DT, 3, QUANT>(a, st);
    case 256: return launch_rq<DT, 4, QUANT>(a, st);
    case 1024: return launch_rq<DT, 5, QUANT>(a, st);
    case 4096: return launch_rq<DT, 6, QUANT>(a, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace

extern "C" {

int ic_smoothrot_prepare(const float* factors, int64_t K, int dtype, float* fdt_out,
                         float* rcp_out, void* stream) {
  if (K < 0 || (K > 0 && (!factors || !fdt_out || !rcp_out)))
    return ic_set_error(IC_ERR_INVALID_ARG, "ic_smoothrot_prepare: bad arguments");
  if (K == 0) return IC_OK;
  hipStream_t st = (hipStream_t)stream;
  dim3 grid((unsigned)((K + 255) / 256)), block(256);
  switch (dtype) {
    case IC_DTYPE_F16: factor_prep_kernel<IC_DTYPE_F16><<<grid, block, 0, st>>>(factors, (int)K, fdt_out, rcp_out); break;
    case IC_DTYPE_BF16: factor_prep_kernel<IC_DTYPE_BF16><<<grid, block, 0, st>>>(factors, (int)K, fdt_out, rcp_out); break;
    case IC_DTYPE_F32: factor_prep_kernel<IC_DTYPE_F32><<<grid, block, 0, st>>>(factors, (int)K, fdt_out, rcp_out); break;
    default: return ic_set_error(IC_ERR_INVALID_ARG, "ic_smoothrot_prepare: dtype must be f16/bf16/f32");
  }
  return ic_check_launch("ic_smoothrot_prepare");
}

static int check_rotq(const ic_rotq_args* a, bool quant, const char* who) {
  if (!a) return ic_set_error(IC_ERR_INVALID_ARG, "%s: null args", who);
  if (a->dtype != IC_DTYPE_F16 && a->dtype != IC_DTYPE_BF16 && a->dtype != IC_DTYPE_F32)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: dtype must be f16/bf16/f32", who);
  if (a->M < 0 || a->K_in <= 0 || a->K_w <= 0 || a->ldx < a->K_in)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: bad shape M=%lld K_in=%lld K_w=%lld ldx=%lld", who,
                        (long long)a->M, (long long)a->K_in, (long long)a->K_w, (long long)a->ldx);
  const int R = a->rot_size;
  if (!(R == 0 || R == 16 || R == 64 || R == 256 || R == 1024 || R == 4096))
    return ic_set_error(IC_ERR_UNSUPPORTED,
                        "%s: rot_size %d unsupported (regular Hadamard sizes 16/64/256/1024/4096 or 0)",
                        who, R);
  const int64_t K_r = R == 0 ? a->K_in : ((a->K_in + R - 1) / R) * R;
  if (a->K_w < K_r)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: K_w=%lld smaller than the rotated width %lld", who,
                        (long long)a->K_w, (long long)K_r);
  if (a->K_w > (int64_t)kTile * kMaxTiles)
    return ic_set_error(IC_ERR_UNSUPPORTED, "%s: K_w=%lld exceeds the fused row limit %d", who,
                        (long long)a->K_w, kTile * kMaxTiles);
  if (a->dtype == IC_DTYPE_F32 && a->K_w > kTile * kMaxTiles / 2)
    return ic_set_error(IC_ERR_UNSUPPORTED, "%s: f32 rows are limited to %d", who, kTile * kMaxTiles / 2);
  if (a->M > 0 && !a->x) return ic_set_error(IC_ERR_INVALID_ARG, "%s: null x", who);
  if ((a->sr_rcp == nullptr) != (a->sr_f == nullptr) || (a->sm_rcp == nullptr) != (a->sm_f == nullptr))
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: factor arrays come in (rcp, f) pairs", who);
  if (a->dtype == IC_DTYPE_F32 && ((a->sr_f && !a->sr_rcp) || (a->sm_f && !a->sm_rcp)))
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: factor arrays come in (rcp, f) pairs", who);
  if (quant) {
    if (a->M > 0 && (!a->q_out || !a->s_out || a->ldq < a->K_w))
      return ic_set_error(IC_ERR_INVALID_ARG, "%s: bad quantized output", who);
  } else {
    if (a->M > 0 && (!a->y_out || a->ldy < a->K_w))
      return ic_set_error(IC_ERR_INVALID_ARG, "%s: bad prepared output", who);
  }
  if (a->M > 0x7fffffffLL) return ic_set_error(IC_ERR_UNSUPPORTED, "%s: M too large", who);
  return IC_OK;
}

static int run_rotq(const ic_rotq_args* a, bool quant, void* stream) {
  const char* who = quant ? "ic_rotate_quantize" : "ic_prepare_activation";
  int rc = check_rotq(a, quant, who);
  if (rc) return rc;
  if (a->M == 0) return IC_OK;
  hipStream_t st = (hipStream_t)stream;
  hipError_t e = hipErrorInvalidValue;
  if (quant && fast_path_ok(*a)) {
    e = a->dtype == IC_DTYPE_F16 ? ic_rq_fast_f16(*a, st) : ic_rq_fast_bf16(*a, st);
    if (e != hipSuccess) return ic_set_error(IC_ERR_LAUNCH, "%s: %s", who, hipGetErrorString(e));
    return IC_OK;
  }
  switch (a->dtype) {
    case IC_DTYPE_F16: e = quant ? dispatch_rot<IC_DTYPE_F16, true>(*a, st) : dispatch_rot<IC_DTYPE_F16, false>(*a, st); break;
    case IC_DTYPE_BF16: e = quant ? dispatch_rot<IC_DTYPE_BF16, true>(*a, st) : dispatch_rot<IC_DTYPE_BF16, false>(*a, st); break;
    case IC_DTYPE_F32: e = quant ? dispatch_rot<IC_DTYPE_F32, true>(*a, st) : dispatch_rot<IC_DTYPE_F32, false>(*a, st); break;
  }
  if (e != hipSuccess) return ic_set_error(IC_ERR_LAUNCH, "%s: %s", who, hipGetErrorString(e));
  return IC_OK;
}

int ic_rotate_quantize(const void* x, int dtype, int64_t M, int64_t K_in, int64_t ldx,
                       const float* sr_rcp, const float* sr_f, int rot_size, int64_t K_w,
                       const int32_t* perm, const float* sm_rcp, const float* sm_f, int8_t* q_out,
                       int64_t ldq, float* s_out, void* stream) {
  ic_rotq_args a{x, dtype, M, K_in, ldx, sr_rcp, sr_f, rot_size, K_w, perm, sm_rcp, sm_f,
                 q_out, ldq, s_out, nullptr, 0};
  return run_rotq(&a, true, stream);
}

int ic_norm_rotate_quantize(const void* x, int dtype, int64_t M, int64_t K_in, int64_t ldx, int norm_kind,
                            const float* weight, const float* bias, float eps, const float* sr_rcp,
                            const float* sr_f, int rot_size, int64_t K_w, const int32_t* perm, int8_t* q_out,
                            int64_t ldq, float* s_out, void* stream) {
  const char* who = "ic_norm_rotate_quantize";
  ic_rotq_args a{x, dtype, M, K_in, ldx, sr_rcp, sr_f, rot_size, K_w, perm, nullptr, nullptr,
                 q_out, ldq, s_out, nullptr, 0, norm_kind, weight, bias, eps};
  if (norm_kind != IC_NORM_LAYER && norm_kind != IC_NORM_RMS)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: norm_kind must be IC_NORM_LAYER or IC_NORM_RMS", who);
  if (!(eps >= 0.0f)) return ic_set_error(IC_ERR_INVALID_ARG, "%s: eps must be >= 0", who);
  int rc = check_rotq(&a, true, who);
  if (rc) return rc;
  if (a.M == 0) return IC_OK;
  auto al16 = [](const void* p) { return (((uintptr_t)p) & 15) == 0; };
  if (!fast_path_ok(a) || !al16(weight) || !al16(bias))
    return ic_set_error(IC_ERR_UNSUPPORTED,
                        "%s: needs f16/bf16 rows with K_in and K_w multiples of 16, K_w <= %d, 16-byte aligned "
                        "rows, factors, perm, weight and bias", who, kTile * kMaxTiles);
  hipStream_t st = (hipStream_t)stream;
  const hipError_t e = dtype == IC_DTYPE_F16 ? ic_rq_norm_f16(a, st) : ic_rq_norm_bf16(a, st);
  if (e != hipSuccess) return ic_set_error(IC_ERR_LAUNCH, "%s: %s", who, hipGetErrorString(e));
  return IC_OK;
}

int ic_prepare_activation(const void* x, int dtype, int64_t M, int64_t K_in, int64_t ldx,
                          const float* sr_rcp, const float* sr_f, int rot_size, int64_t K_w,
                          const int32_t* perm, const float* sm_rcp, const float* sm_f,
                          void* y_out, int64_t ldy, void* stream) {
  ic_rotq_args a{x, dtype, M, K_in, ldx, sr_rcp, sr_f, rot_size, K_w, perm, sm_rcp, sm_f,
                 nullptr, 0, nullptr, y_out, ldy};
  return run_rotq(&a, false, stream);
}

int64_t ic_max_fused_row(void) { return (int64_t)kTile * kMaxTiles; }

int ic_permute_quantize(const void* y, int dtype, int64_t M, int64_t K_y, int64_t ldy, int64_t K_w,
                        const int32_t* perm, const float* sm_rcp, const float* sm_f, int8_t* q_out, int64_t ldq,
                        float* s_out, void* out, int64_t ldo, void* stream) {
  const char* who = "ic_permute_quantize";
  if (dtype != IC_DTYPE_F16 && dtype != IC_DTYPE_BF16 && dtype != IC_DTYPE_F32)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: dtype must be f16/bf16/f32", who);
  if (M < 0 || K_y <= 0 || K_w < K_y || ldy < K_y || K_w > 0x7fffffffLL || M > 0x7fffffffLL)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: bad shape M=%lld K_y=%lld K_w=%lld ldy=%lld", who, (long long)M,
                        (long long)K_y, (long long)K_w, (long long)ldy);
  if ((sm_rcp == nullptr) != (sm_f == nullptr))
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: factor arrays come in (rcp, f) pairs", who);
  const bool quant = q_out != nullptr || s_out != nullptr;
  if (quant == (out != nullptr))
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: give either q_out and s_out or out", who);
  if (M == 0) return IC_OK;
  if (!y || (quant && (!q_out || !s_out || ldq < K_w)) || (!quant && ldo < K_w))
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: bad pointers or output stride", who);
  hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  switch (dtype) {
    case IC_DTYPE_F16:
      e = launch_permute_rows<IC_DTYPE_F16>(y, ldy, M, K_y, K_w, perm, sm_rcp, sm_f, q_out, ldq, s_out, out, ldo, st);
      break;
    case IC_DTYPE_BF16:
      e = launch_permute_rows<IC_DTYPE_BF16>(y, ldy, M, K_y, K_w, perm, sm_rcp, sm_f, q_out, ldq, s_out, out, ldo, st);
      break;
    default:
      e = launch_permute_rows<IC_DTYPE_F32>(y, ldy, M, K_y, K_w, perm, sm_rcp, sm_f, q_out, ldq, s_out, out, ldo, st);
      break;
  }
  if (e != hipSuccess) return ic_set_error(IC_ERR_LAUNCH, "%s: %s", who, hipGetErrorString(e));
  return IC_OK;
}

int ic_dynamic_quantize(const void* x, int dtype, int64_t M, int64_t K, int64_t ldx, int8_t* q_out,
                        int64_t ldq, float* s_out, void* stream) {
  if (M < 0 || K <= 0 || ldx < K || ldq < K || (M > 0 && (!x || !q_out || !s_out)))
    return ic_set_error(IC_ERR_INVALID_ARG, "ic_dynamic_quantize: bad arguments");
  if (dtype != IC_DTYPE_F16 && dtype != IC_DTYPE_BF16 && dtype != IC_DTYPE_F32)
    return ic_set_error(IC_ERR_INVALID_ARG, "ic_dynamic_quantize: dtype must be f16/bf16/f32");
  if (M == 0) return IC_OK;
  hipStream_t st = (hipStream_t)stream;
  const int64_t lim = dtype == IC_DTYPE_F32 ? kTile * kMaxTiles / 2 : kTile * kMaxTiles;
  if (K <= lim)
    return ic_rotate_quantize(x, dtype, M, K, ldx, nullptr, nullptr, 0, K, nullptr, nullptr, nullptr,
                              q_out, ldq, s_out, stream);
  switch (dtype) {
    case IC_DTYPE_F16: quant_rows_kernel<IC_DTYPE_F16><<<dim3((unsigned)M), dim3(kThreads), 0, st>>>(x, ldx, (int)K, q_out, ldq, s_out); break;
    case IC_DTYPE_BF16: quant_rows_kernel<IC_DTYPE_BF16><<<dim3((unsigned)M), dim3(kThreads), 0, st>>>(x, ldx, (int)K, q_out, ldq, s_out); break;
    default: quant_rows_kernel<IC_DTYPE_F32><<<dim3((unsigned)M), dim3(kThreads), 0, st>>>(x, ldx, (int)K, q_out, ldq, s_out); break;
  }
  return ic_check_launch("ic_dynamic_quantize");
}

}  // extern "C"
