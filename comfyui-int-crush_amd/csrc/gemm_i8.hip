// INT8 / packed-INT4 MFMA GEMM entry points (kernels in gemm_i8.h; the
// epilogue-option instantiations compile in gemm_i8_epi.hip).
#include <mutex>

#include "gemm_i8.h"

namespace {

// Split-K scratch of ic_gemm_w4a8_noalloc: one array per device, loaded with
// the code object and held until the process ends.  Host code never passes
// `scratch` itself to a kernel (on the host the name is only a stand-in for
// the symbol); it uses the device address hipGetSymbolAddress returns, looked
// up once per device with that device current and kept in scratch_ptr.
constexpr int64_t kScratchBytes = IC_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex scratch_mu;
void* scratch_ptr[kMaxDevices];

int scratch_for_current_device(void** out, const char* who) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return ic_set_error(IC_ERR_LAUNCH, "%s: hipGetDevice: %s", who, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return ic_set_error(IC_ERR_UNSUPPORTED, "%s: device %d beyond the %d supported", who, dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return ic_set_error(IC_ERR_LAUNCH, "%s: hipGetSymbolAddress(scratch) on device %d: %s", who, dev,
                          hipGetErrorString(e));
    scratch_ptr[dev] = p;
  }
  *out = scratch_ptr[dev];
  return IC_OK;
}

int run_gemm(GemmArgs g, hipStream_t st, const char* who, bool force_generic) {
  if (g.epi.act != 0 || g.epi.res != nullptr) return ic_gemm_run_epi(g, st, who, force_generic);
  return run_gemm_t<false>(g, st, who, force_generic);
}

// W4A8 on either nibble order of the packed weights (kil: K-interleaved);
// M <= 16 takes the GEMV where its shape and groups allow.
int gemm_w4a8_any(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const uint8_t* w, int64_t N, int64_t ldw,
                  const float* s_w, int64_t num_groups, const float* s_a, const void* bias, int bias_dtype,
                  int activation, const void* residual, int residual_dtype, int64_t ldr, void* out, int out_dtype,
                  int64_t ldo, void* workspace, int64_t workspace_bytes, void* stream, bool kil, const char* who) {
  if (int rc = ic_check_epi(who, activation, residual, residual_dtype, ldr, N)) return rc;
  const ic_epi epi{activation, residual, residual_dtype, ldr};
  if (ic_gemv_applicable(M, K, xq, ldx, w, ldw) && ldw * 2 >= K && N > 0 && ldo >= N && ldx >= K &&
      ic_gemv_w4a8_groups_ok(M, K, num_groups))
    return ic_gemv_w4a8_epi(xq, M, K, ldx, w, N, ldw, s_w, num_groups, s_a, bias, bias_dtype, out, out_dtype, ldo, epi,
                            stream, kil ? kW4Kil : kW4Plain);
  GemmArgs g{xq, ldx, w, ldw, s_a, s_w, (int)num_groups, bias, bias_dtype, out, out_dtype,
             ldo, (int)M, (int)N, (int)K, nullptr, true, workspace, workspace_bytes, epi, kil};
  return run_gemm(g, (hipStream_t)stream, who, false);
}

}  // namespace

// Validation shared by the _ex entry points: activation code and residual.
int ic_check_epi(const char* who, int activation, const void* residual, int residual_dtype, int64_t ldr,
                 int64_t N) {
  if (activation < 0 || activation > 3)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: activation must be 0 (none), 1 (SiLU), 2 (GELU) or 3 (GELU tanh)",
                        who);
  if (residual != nullptr && residual_dtype != IC_DTYPE_F16 && residual_dtype != IC_DTYPE_BF16 &&
      residual_dtype != IC_DTYPE_F32)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: residual dtype must be f16/bf16/f32", who);
  if (residual != nullptr && ldr < N)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: residual row stride %lld < N=%lld", who, (long long)ldr,
                        (long long)N);
  return IC_OK;
}

extern "C" {

int ic_init_device(void) {
  void* p = nullptr;
  return scratch_for_current_device(&p, "ic_init_device");
}

int64_t ic_gemm_splitk_bytes(int64_t M, int64_t N, int64_t K, int64_t num_groups, int int4) {
  if (M <= IC_GEMV_MAX_M || N <= 0 || K <= 0 || K % kBK != 0 || num_groups < 1) return 0;
  if (num_groups > 1 && (K % num_groups != 0 || (K / num_groups) % 128 != 0)) return 0;
  if (M * N > (1LL << 31)) return 0;
  GemmArgs g{nullptr, K, nullptr, K, nullptr, nullptr, (int)num_groups, nullptr, 0, nullptr, IC_DTYPE_F32,
             N, (int)M, (int)N, (int)K, nullptr, int4 != 0};
  const int S = splitk_plan(g, num_groups > 1);
  return S > 1 ? (int64_t)S * M * N * 4 : 0;
}

int ic_gemm_w8a8_ex(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const int8_t* w, int64_t N, int64_t ldw,
                    const float* s_a, const float* s_w, const void* bias, int bias_dtype, int activation,
                    const void* residual, int residual_dtype, int64_t ldr, void* out, int out_dtype, int64_t ldo,
                    void* workspace, int64_t workspace_bytes, void* stream) {
  if (int rc = ic_check_epi("ic_gemm_w8a8", activation, residual, residual_dtype, ldr, N)) return rc;
  const ic_epi epi{activation, residual, residual_dtype, ldr};
  if (ic_gemv_applicable(M, K, xq, ldx, w, ldw) && ldw >= K && N > 0 && ldo >= N && ldx >= K)
    return ic_gemv_w8a8_epi(xq, M, K, ldx, w, N, ldw, s_a, s_w, bias, bias_dtype, out, out_dtype, ldo, epi, stream);
  GemmArgs g{xq, ldx, (const uint8_t*)w, ldw, s_a, s_w, 1, bias, bias_dtype, out, out_dtype, ldo,
             (int)M, (int)N, (int)K, nullptr, false, workspace, workspace_bytes, epi};
  return run_gemm(g, (hipStream_t)stream, "ic_gemm_w8a8", false);
}

int ic_gemm_w8a8_ws(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const int8_t* w, int64_t N,
                    int64_t ldw, const float* s_a, const float* s_w, const void* bias, int bias_dtype,
                    void* out, int out_dtype, int64_t ldo, void* workspace, int64_t workspace_bytes,
                    void* stream) {
  return ic_gemm_w8a8_ex(xq, M, K, ldx, w, N, ldw, s_a, s_w, bias, bias_dtype, 0, nullptr, 0, 0, out, out_dtype, ldo,
                         workspace, workspace_bytes, stream);
}

int ic_gemm_w8a8(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const int8_t* w, int64_t N,
                 int64_t ldw, const float* s_a, const float* s_w, const void* bias, int bias_dtype,
                 void* out, int out_dtype, int64_t ldo, void* stream) {
  return ic_gemm_w8a8_ws(xq, M, K, ldx, w, N, ldw, s_a, s_w, bias, bias_dtype, out, out_dtype, ldo, nullptr, 0,
                         stream);
}

int ic_gemm_w4a8_ex(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const uint8_t* w_packed, int64_t N,
                    int64_t ldw, const float* s_w, int64_t num_groups, const float* s_a, const void* bias,
                    int bias_dtype, int activation, const void* residual, int residual_dtype, int64_t ldr, void* out,
                    int out_dtype, int64_t ldo, void* workspace, int64_t workspace_bytes, void* stream) {
  return gemm_w4a8_any(xq, M, K, ldx, w_packed, N, ldw, s_w, num_groups, s_a, bias, bias_dtype, activation, residual,
                       residual_dtype, ldr, out, out_dtype, ldo, workspace, workspace_bytes, stream, false,
                       "ic_gemm_w4a8");
}

int ic_gemm_w4a8_kil_ex(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const uint8_t* w_kil, int64_t N,
                        int64_t ldw, const float* s_w, int64_t num_groups, const float* s_a, const void* bias,
                        int bias_dtype, int activation, const void* residual, int residual_dtype, int64_t ldr,
                        void* out, int out_dtype, int64_t ldo, void* workspace, int64_t workspace_bytes,
                        void* stream) {
  if (K % 8 != 0)
    return ic_set_error(IC_ERR_INVALID_ARG, "ic_gemm_w4a8_kil_ex: K=%lld must be a multiple of 8", (long long)K);
  return gemm_w4a8_any(xq, M, K, ldx, w_kil, N, ldw, s_w, num_groups, s_a, bias, bias_dtype, activation, residual,
                       residual_dtype, ldr, out, out_dtype, ldo, workspace, workspace_bytes, stream, true,
                       "ic_gemm_w4a8_kil_ex");
}

int ic_gemm_w4a8_unpacked_ex(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const int8_t* w, int64_t N,
                             int64_t ldw, const float* s_w, int64_t num_groups, const float* s_a, const void* bias,
                             int bias_dtype, int activation, const void* residual, int residual_dtype, int64_t ldr,
                             void* out, int out_dtype, int64_t ldo, void* workspace, int64_t workspace_bytes,
                             void* stream) {
  const char* who = "ic_gemm_w4a8_unpacked_ex";
  if (int rc = ic_check_epi(who, activation, residual, residual_dtype, ldr, N)) return rc;
  const ic_epi epi{activation, residual, residual_dtype, ldr};
  GemmArgs g{xq, ldx, (const uint8_t*)w, ldw, s_a, s_w, (int)num_groups, bias, bias_dtype, out, out_dtype,
             ldo, (int)M, (int)N, (int)K, nullptr, false, workspace, workspace_bytes, epi};
  return run_gemm(g, (hipStream_t)stream, who, false);
}

int ic_gemm_w4a8_ws(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const uint8_t* w_packed,
                    int64_t N, int64_t ldw, const float* s_w, int64_t num_groups, const float* s_a,
                    const void* bias, int bias_dtype, void* out, int out_dtype, int64_t ldo,
                    void* workspace, int64_t workspace_bytes, void* stream) {
  return ic_gemm_w4a8_ex(xq, M, K, ldx, w_packed, N, ldw, s_w, num_groups, s_a, bias, bias_dtype, 0, nullptr, 0, 0,
                         out, out_dtype, ldo, workspace, workspace_bytes, stream);
}

int ic_gemm_w4a8(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const uint8_t* w_packed,
                 int64_t N, int64_t ldw, const float* s_w, int64_t num_groups, const float* s_a,
                 const void* bias, int bias_dtype, void* out, int out_dtype, int64_t ldo,
                 void* stream) {
  return ic_gemm_w4a8_ws(xq, M, K, ldx, w_packed, N, ldw, s_w, num_groups, s_a, bias, bias_dtype, out, out_dtype,
                         ldo, nullptr, 0, stream);
}

int ic_gemm_w4a8_noalloc(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const uint8_t* w_packed, int64_t N,
                         int64_t ldw, const float* s_w, int64_t num_groups, const float* s_a, const void* bias,
                         int bias_dtype, void* out, int out_dtype, int64_t ldo, void* stream) {
  const char* who = "ic_gemm_w4a8_noalloc";
  const int64_t need = ic_gemm_splitk_bytes(M, N, K, num_groups, 1);
  if (need > kScratchBytes)
    return ic_set_error(IC_ERR_UNSUPPORTED,
                        "%s: M=%lld N=%lld K=%lld splits K over %lld bytes of partials, above the %lld-byte static "
                        "scratch; use ic_gemm_w4a8_ws with a workspace",
                        who, (long long)M, (long long)N, (long long)K, (long long)need, (long long)kScratchBytes);
  void* ws = nullptr;
  if (need > 0) {
    if (int rc = scratch_for_current_device(&ws, who)) return rc;
  }
  return ic_gemm_w4a8_ex(xq, M, K, ldx, w_packed, N, ldw, s_w, num_groups, s_a, bias, bias_dtype, 0, nullptr, 0, 0,
                         out, out_dtype, ldo, ws, need, stream);
}

int ic_gemm_w8a8_acc_i32(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const int8_t* w,
                         int64_t N, int64_t ldw, int32_t* acc, int generic, void* stream) {
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
