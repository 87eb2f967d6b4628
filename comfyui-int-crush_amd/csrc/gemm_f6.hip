// Entry points of the grouped W4A8 GEMM on e3m2 operands (kernel and formats
// in gemm_f6.h): the two format conversions and the GEMM.  An alternative to
// ic_gemm_w4a8's grouped path with bit-identical outputs; the library's own
// routing does not use it (it measured level with the int8 kernel, being
// bound by LDS reads where the int8 kernel is bound by VALU issue).
#include "gemm_f6.h"
#include "gemm_i8.h"

namespace {

int64_t f6_stages(int64_t K) { return K > 0 && K % 128 == 0 ? K / 128 : 0; }

template <int OUT_DT, int TMB>
hipError_t launch_f6_t(const GemmArgs& g, const uint8_t* a6, const uint8_t* w6, int64_t a_rb, int64_t b_cb,
                       hipStream_t st) {
  using RT = f6::Rows<TMB>;
  const int tiles = ((g.M + RT::BM - 1) / RT::BM) * ((g.N + f6::BN - 1) / f6::BN);
  auto kern = gemm_w4a8f6_kernel<OUT_DT, false, TMB>;
  constexpr size_t shm = RT::lds_bytes;
  static unsigned char lds_set[64];  // per device
  if (hipError_t e = ic_set_lds_limit((const void*)kern, (int)shm, lds_set)) return e;
  kern<<<dim3(tiles), dim3(kNT), shm, st>>>(a6, a_rb, w6, b_cb, g.s_a, g.s_w, g.G, g.bias, g.bias_dt, g.C, g.ldc,
                                            g.M, g.N, g.K, g.epi);
  return hipGetLastError();
}

template <int OUT_DT>
hipError_t launch_f6(const GemmArgs& g, const uint8_t* a6, const uint8_t* w6, int64_t a_rb, int64_t b_cb,
                     hipStream_t st) {
  // the row count of the int8 big-tile kernel for the same shape
  switch (big_rows(g)) {
    case 8: return launch_f6_t<OUT_DT, 8>(g, a6, w6, a_rb, b_cb, st);
    case 10: return launch_f6_t<OUT_DT, 10>(g, a6, w6, a_rb, b_cb, st);
    default: return launch_f6_t<OUT_DT, 9>(g, a6, w6, a_rb, b_cb, st);
  }
}

}  // namespace

extern "C" {

int64_t ic_f6_activation_bytes(int64_t M, int64_t K) {
  const int64_t s = f6_stages(K);
  return M > 0 && s > 0 ? (M + 15) / 16 * s * 3072 : 0;
}

int64_t ic_f6_weight_bytes(int64_t N, int64_t K) {
  const int64_t s = f6_stages(K);
  return N > 0 && s > 0 ? (N + 15) / 16 * s * 1536 : 0;
}

int ic_f6_split_activations(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, uint8_t* a6, void* stream) {
  const char* who = "ic_f6_split_activations";
  if (M < 0 || f6_stages(K) == 0 || ldx < K || (ldx & 15) || M > INT32_MAX / 2)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: needs K a positive multiple of 128 and a row stride >= K, "
                        "a multiple of 16 (M=%lld K=%lld ldx=%lld)", who, (long long)M, (long long)K,
                        (long long)ldx);
  if (M == 0) return IC_OK;
  if (!xq || !a6 || ((uintptr_t)xq & 15) || ((uintptr_t)a6 & 15))
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: null or unaligned (16-byte) pointer", who);
  const int64_t threads = M * (K / 16);
  split_a6_kernel<<<dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, (hipStream_t)stream>>>(
      xq, ldx, a6, f6_stages(K) * 3072, (int)M, (int)K);
  return ic_check_launch(who);
}

int ic_f6_repack_weights(const uint8_t* w_packed, int64_t N, int64_t K, int64_t ldw, uint8_t* w6, void* stream) {
  const char* who = "ic_f6_repack_weights";
  if (N <= 0 || f6_stages(K) == 0 || ldw * 2 < K || (ldw & 15) || N > INT32_MAX / 2)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: needs N > 0, K a positive multiple of 128 and a row stride "
                        ">= K/2 bytes, a multiple of 16 (N=%lld K=%lld ldw=%lld)", who, (long long)N,
                        (long long)K, (long long)ldw);
  if (!w_packed || !w6 || ((uintptr_t)w_packed & 15) || ((uintptr_t)w6 & 15))
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: null or unaligned (16-byte) pointer", who);
  const int64_t threads = N * (K / 32);
  repack_w6_kernel<<<dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, (hipStream_t)stream>>>(
      w_packed, ldw, w6, f6_stages(K) * 1536, (int)N, (int)K);
  return ic_check_launch(who);
}

int ic_gemm_w4a8_f6(const uint8_t* a6, int64_t M, int64_t K, const uint8_t* w6, int64_t N, const float* s_w,
                    int64_t num_groups, const float* s_a, const void* bias, int bias_dtype, void* out,
                    int out_dtype, int64_t ldo, void* stream) {
  const char* who = "ic_gemm_w4a8_f6";
  if (M < 0 || N <= 0 || f6_stages(K) == 0 || num_groups < 2 || K % num_groups != 0 ||
      (K / num_groups) % 128 != 0)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: needs K a multiple of 128 and groups of a multiple of 128 "
                        "columns, at least two (M=%lld N=%lld K=%lld num_groups=%lld)", who, (long long)M,
                        (long long)N, (long long)K, (long long)num_groups);
  if (out_dtype != IC_DTYPE_F16 && out_dtype != IC_DTYPE_BF16)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: out dtype must be f16 or bf16", who);
  if (bias && bias_dtype != IC_DTYPE_F16 && bias_dtype != IC_DTYPE_BF16 && bias_dtype != IC_DTYPE_F32)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: bias dtype must be f16/bf16/f32", who);
  if (ldo < N || (ldo & 7) || (N & 7) || ldo >= (1LL << 24) || M > INT32_MAX / 2 || N > INT32_MAX / 2 ||
      N * num_groups * 4 >= (1LL << 31) || f6_stages(K) * 1536 * 16 >= (1LL << 31))
    return ic_set_error(IC_ERR_UNSUPPORTED, "%s: needs N and the output row stride multiples of 8 "
                        "(N=%lld ldo=%lld) and the 32-bit offsets of its DMAs", who, (long long)N, (long long)ldo);
  if (M == 0) return IC_OK;
  if (!a6 || !w6 || !s_w || !s_a || !out || ((uintptr_t)a6 & 15) || ((uintptr_t)w6 & 15) || ((uintptr_t)out & 15))
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: null or unaligned (16-byte) pointer", who);
  GemmArgs g{nullptr, K, nullptr, K / 2, s_a, s_w, (int)num_groups, bias, bias_dtype, out, out_dtype, ldo,
             (int)M, (int)N, (int)K, nullptr, true};
  const int64_t a_rb = f6_stages(K) * 3072, b_cb = f6_stages(K) * 1536;
  hipError_t e = out_dtype == IC_DTYPE_F16 ? launch_f6<IC_DTYPE_F16>(g, a6, w6, a_rb, b_cb, (hipStream_t)stream)
                                           : launch_f6<IC_DTYPE_BF16>(g, a6, w6, a_rb, b_cb, (hipStream_t)stream);
  if (e != hipSuccess) return ic_set_error(IC_ERR_LAUNCH, "%s: %s", who, hipGetErrorString(e));
  return IC_OK;
}

}  // extern "C"
