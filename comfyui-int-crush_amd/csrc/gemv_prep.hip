// Entry points of the single-launch prep + GEMV (kernels in gemv_prep.h):
// argument checks and the choice of instantiation.
#include <algorithm>

#include "gemv_prep.h"

namespace {

int rot_log4(int R) {
  switch (R) {
    case 0: return 0;
    case 16: return 2;
    case 64: return 3;
    case 256: return 4;
    case 1024: return 5;
    case 4096: return 6;
  }
  return -1;
}

// Checks shared by both weight formats; fills the launch description's
// preparation and output fields.  w_row_bytes: bytes of K weights of a row.
int prep_gemv_setup(const char* who, const void* x, int dtype, int64_t M, int64_t K_in, int64_t ldx,
                    const float* sr_rcp, const float* sr_f, int rot_size, const int32_t* perm, const float* sm_rcp,
                    const float* sm_f, const void* w, int64_t N, int64_t K, int64_t ldw_bytes, int64_t w_row_bytes,
                    const float* s_w, const void* bias, int bias_dtype, int activation, const void* residual,
                    int residual_dtype, int64_t ldr, void* out, int out_dtype, int64_t ldo,
                    gemvp::PrepGemvLaunch& L) {
  if (dtype != IC_DTYPE_F16 && dtype != IC_DTYPE_BF16)
    return ic_set_error(IC_ERR_UNSUPPORTED, "%s: activation dtype must be f16/bf16 (f32 rows: ic_rotate_quantize, "
                        "then the GEMV)", who);
  if (M < 0 || M > IC_GEMV_MAX_M)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: M=%lld outside [0, %d]", who, (long long)M, IC_GEMV_MAX_M);
  if (K_in <= 0 || ldx < K_in || N <= 0 || N > 0x7fffffffLL || ldo < N || K <= 0)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: bad shape K_in=%lld ldx=%lld N=%lld K=%lld ldo=%lld", who,
                        (long long)K_in, (long long)ldx, (long long)N, (long long)K, (long long)ldo);
  if (K % 128 != 0 || K > IC_PREP_GEMV_MAX_K || M * K > IC_PREP_GEMV_MAX_CODES)
    return ic_set_error(IC_ERR_UNSUPPORTED, "%s: K=%lld must be a multiple of 128, <= %d, and M*K <= %d", who,
                        (long long)K, IC_PREP_GEMV_MAX_K, IC_PREP_GEMV_MAX_CODES);
  const int log4r = rot_log4(rot_size);
  if (log4r < 0)
    return ic_set_error(IC_ERR_UNSUPPORTED,
                        "%s: rot_size %d unsupported (regular Hadamard sizes 16/64/256/1024/4096 or 0)", who, rot_size);
  const int64_t K_r = rot_size == 0 ? K_in : ((K_in + rot_size - 1) / rot_size) * rot_size;
  if (K < K_r)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: K=%lld smaller than the rotated width %lld", who, (long long)K,
                        (long long)K_r);
  if ((sr_rcp == nullptr) != (sr_f == nullptr) || (sm_rcp == nullptr) != (sm_f == nullptr))
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: factor arrays come in (rcp, f) pairs", who);
  auto al16 = [](const void* p) { return (((uintptr_t)p) & 15) == 0; };
  if (K_in % 16 != 0 || (ldx * 2) % 16 != 0 || !al16(x) || !al16(sr_rcp) || !al16(perm) || !al16(sm_rcp))
    return ic_set_error(IC_ERR_UNSUPPORTED, "%s: needs K_in a multiple of 16, ldx a multiple of 8 and 16-byte "
                        "aligned rows, factors and perm", who);
  if (bias && bias_dtype != IC_DTYPE_F16 && bias_dtype != IC_DTYPE_BF16 && bias_dtype != IC_DTYPE_F32)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: bias dtype must be f16/bf16/f32", who);
  if (out_dtype != IC_DTYPE_F16 && out_dtype != IC_DTYPE_BF16 && out_dtype != IC_DTYPE_F32)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: out dtype must be f16/bf16/f32", who);
  if (int rc = ic_check_epi(who, activation, residual, residual_dtype, ldr, N)) return rc;
  if (M > 0 && (!x || !w || !s_w || !out)) return ic_set_error(IC_ERR_INVALID_ARG, "%s: null pointer", who);
  if (ldw_bytes < w_row_bytes || ((uintptr_t)w & 15) != 0 || (ldw_bytes & 15) != 0)
    return ic_set_error(IC_ERR_UNSUPPORTED, "%s: weights must be 16-byte aligned with a row stride of at least K "
                        "values, a multiple of 16 bytes", who);
  L.pa = gemvp::PrepArgs{x, ldx, (int)K_in, (int)K_r, sr_rcp, sr_f, perm, sm_rcp, sm_f};
  L.log4r = log4r;
  L.B = (const uint8_t*)w;
  L.ldb = ldw_bytes;
  L.s_w = s_w;
  L.bias = bias;
  L.bias_dt = bias_dtype;
  L.C = out;
  L.out_dt = out_dtype;
  L.ldc = ldo;
  L.M = (int)M;
  L.N = (int)N;
  L.K = (int)K;
  L.epi = ic_epi{activation, residual, residual_dtype, ldr};
  return IC_OK;
}

int prep_gemv_launch(const char* who, int dtype, gemvp::PrepGemvLaunch& L, void* stream) {
  if (L.M == 0) return IC_OK;
  // at most one workgroup per CU, as long as a wave's loads fit its
  // registers and the block sums of the workgroup's column blocks the 36 KB
  // tbuf area
  const int nblk = (L.N + 15) / 16, cus = ic_num_cus();
  const int64_t sums = (L.int4 && L.grouped ? L.K / 128 : 4) * (int64_t)L.M * 16 * 4;
  const int fit_lds = (int)((int64_t)rq::kTbufDoubles * 8 / sums);
  const int steps = (L.K / 128 + 3) / 4;
  const int fit_regs = (L.int4 ? gemvp::kPrepGemvSteps<true> : gemvp::kPrepGemvSteps<false>) / steps;
  L.cbs = std::max(1, std::min({(nblk + cus - 1) / cus, fit_lds, fit_regs}));
  hipStream_t st = (hipStream_t)stream;
  const bool one_tile = L.K <= rq::kTile;
  hipError_t e;
  if (dtype == IC_DTYPE_F16) e = one_tile ? ic_prep_gemv_f16_t1(L, st) : ic_prep_gemv_f16_t2(L, st);
  else e = one_tile ? ic_prep_gemv_bf16_t1(L, st) : ic_prep_gemv_bf16_t2(L, st);
  if (e != hipSuccess) return ic_set_error(IC_ERR_LAUNCH, "%s: %s", who, hipGetErrorString(e));
  return IC_OK;
}

}  // namespace

static_assert(IC_PREP_GEMV_MAX_K == rq::kTile * gemvp::kPrepGemvMaxTiles, "row limit of the instantiations");
static_assert(IC_PREP_GEMV_MAX_CODES == gemv::kXlBytes, "codes held in LDS");
static_assert((IC_PREP_GEMV_MAX_K / 128 + 3) / 4 <= gemvp::kPrepGemvSteps<false>,
              "one column block's steps of a wave fit its registers");

extern "C" {

int ic_prep_gemv_w4a8(const void* x, int dtype, int64_t M, int64_t K_in, int64_t ldx, const float* sr_rcp,
                      const float* sr_f, int rot_size, const int32_t* perm, const float* sm_rcp, const float* sm_f,
                      const uint8_t* w_packed, int64_t N, int64_t K, int64_t ldw, const float* s_w,
                      int64_t num_groups, const void* bias, int bias_dtype, int activation, const void* residual,
                      int residual_dtype, int64_t ldr, void* out, int out_dtype, int64_t ldo, void* stream) {
  const char* who = "ic_prep_gemv_w4a8";
  gemvp::PrepGemvLaunch L{};
  if (int rc = prep_gemv_setup(who, x, dtype, M, K_in, ldx, sr_rcp, sr_f, rot_size, perm, sm_rcp, sm_f, w_packed, N,
                               K, ldw, (K + 1) / 2, s_w, bias, bias_dtype, activation, residual, residual_dtype, ldr,
                               out, out_dtype, ldo, L))
    return rc;
  if (num_groups < 1 || (num_groups > 1 && num_groups * 128 != K))
    return ic_set_error(IC_ERR_UNSUPPORTED, "%s: num_groups must be 1 or K/128", who);
  L.int4 = true;
  L.grouped = num_groups > 1;
  L.G = (int)num_groups;
  return prep_gemv_launch(who, dtype, L, stream);
}

int ic_prep_gemv_w8a8(const void* x, int dtype, int64_t M, int64_t K_in, int64_t ldx, const float* sr_rcp,
                      const float* sr_f, int rot_size, const int32_t* perm, const float* sm_rcp, const float* sm_f,
                      const int8_t* w, int64_t N, int64_t K, int64_t ldw, const float* s_w, const void* bias,
                      int bias_dtype, int activation, const void* residual, int residual_dtype, int64_t ldr,
                      void* out, int out_dtype, int64_t ldo, void* stream) {
  const char* who = "ic_prep_gemv_w8a8";
  gemvp::PrepGemvLaunch L{};
  if (int rc = prep_gemv_setup(who, x, dtype, M, K_in, ldx, sr_rcp, sr_f, rot_size, perm, sm_rcp, sm_f, w, N, K, ldw,
                               K, s_w, bias, bias_dtype, activation, residual, residual_dtype, ldr, out, out_dtype,
                               ldo, L))
    return rc;
  L.int4 = false;
  L.grouped = false;
  L.G = 1;
  return prep_gemv_launch(who, dtype, L, stream);
}

}  // extern "C"
