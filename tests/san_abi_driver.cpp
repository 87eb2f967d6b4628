// Runs the argument validation of every entry point of the C ABI
// (include/intcrush.h) under AddressSanitizer and UndefinedBehaviorSanitizer.
// tests/test_sanitizers.py links it against the library's host code built
// with both sanitizers (--cuda-host-only: the kernels are not compiled, and
// no call below reaches a launch).  Also the pure host planning functions.
// Exit status 0 = every call returned the expected code.
#include <cstdio>

#include "../include/intcrush.h"

static int failures = 0;
static void expect(bool ok, const char* what) {
  if (!ok) {
    std::fprintf(stderr, "FAILED: %s (%s)\n", what, ic_last_error());
    ++failures;
  }
}
#define EXPECT_ERR(call) expect((call) == IC_ERR_INVALID_ARG || (call) == IC_ERR_UNSUPPORTED, #call)
#define EXPECT_OK(call) expect((call) == IC_OK, #call)

int main() {
  expect(ic_version() != nullptr, "ic_version");
  expect(ic_max_fused_row() == 16384, "ic_max_fused_row");
  // prep entry points: bad dtype, rot size, widths, fused-row limit
  EXPECT_ERR(ic_rotate_quantize(nullptr, 7, 1, 16, 16, nullptr, nullptr, 0, 16, nullptr, nullptr, nullptr, nullptr,
                                16, nullptr, nullptr));
  EXPECT_ERR(ic_rotate_quantize(nullptr, 0, 1, 32, 32, nullptr, nullptr, 32, 32, nullptr, nullptr, nullptr, nullptr,
                                32, nullptr, nullptr));
  EXPECT_ERR(ic_rotate_quantize(nullptr, 0, 1, 100, 100, nullptr, nullptr, 64, 100, nullptr, nullptr, nullptr,
                                nullptr, 128, nullptr, nullptr));
  EXPECT_ERR(ic_prepare_activation(nullptr, 0, 1, 20000, 20000, nullptr, nullptr, 0, 20000, nullptr, nullptr,
                                   nullptr, nullptr, 20000, nullptr));
  EXPECT_ERR(ic_permute_quantize(nullptr, 0, 1, 64, 64, 32, nullptr, nullptr, nullptr, nullptr, 64, nullptr,
                                 nullptr, 64, nullptr));
  EXPECT_ERR(ic_dynamic_quantize(nullptr, 9, 1, 64, 64, nullptr, 64, nullptr, nullptr));
  EXPECT_ERR(ic_norm_quantize(nullptr, 0, 1, 64, 64, 9, nullptr, nullptr, 1e-6f, nullptr, 64, nullptr, nullptr));
  EXPECT_ERR(ic_norm_rotate_quantize(nullptr, 2, 1, 64, 64, IC_NORM_LAYER, nullptr, nullptr, 1e-6f, nullptr,
                                     nullptr, 16, 64, nullptr, nullptr, 64, nullptr, nullptr));
  EXPECT_ERR(ic_smoothrot_prepare(nullptr, -1, 0, nullptr, nullptr, nullptr));
  // GEMMs: shape, groups, dtypes, strides, epilogue codes
  EXPECT_ERR(ic_gemm_w4a8(nullptr, 1, 100, 100, nullptr, 4, 50, nullptr, 3, nullptr, nullptr, 0, nullptr, 0, 4,
                          nullptr));
  EXPECT_ERR(ic_gemm_w8a8(nullptr, 64, 128, 64, nullptr, 64, 128, nullptr, nullptr, nullptr, 0, nullptr, 0, 64,
                          nullptr));
  EXPECT_ERR(ic_gemm_w8a8(nullptr, 64, 128, 128, nullptr, 64, 128, nullptr, nullptr, nullptr, 0, nullptr, 5, 64,
                          nullptr));
  EXPECT_ERR(ic_gemm_w8a8_ex(nullptr, 64, 128, 128, nullptr, 64, 128, nullptr, nullptr, nullptr, 0, 9, nullptr, 0,
                             0, nullptr, 0, 64, nullptr, 0, nullptr));
  EXPECT_ERR(ic_gemm_w4a8_ex(nullptr, 64, 128, 128, nullptr, 64, 64, nullptr, 1, nullptr, nullptr, 0, 0,
                             (const void*)16, 7, 64, nullptr, 0, 64, nullptr, 0, nullptr));
  EXPECT_ERR(ic_gemm_w4a16(nullptr, 2, 1, 64, 64, nullptr, 4, 32, nullptr, 1, nullptr, 0, nullptr, 4, nullptr));
  EXPECT_ERR(ic_gemm_w4a16(nullptr, 0, 64, 100, 100, nullptr, 4, 50, nullptr, 3, nullptr, 0, nullptr, 4, nullptr));
  EXPECT_ERR(ic_gemm_w8a8_chain(nullptr, 64, 128, 128, nullptr, 64, 128, nullptr, nullptr, nullptr, 0, 0, nullptr,
                                nullptr, 32, nullptr, 0, 64, nullptr));
  EXPECT_ERR(ic_gemm_w4a8_chain(nullptr, 64, 128, 128, nullptr, 64, 64, nullptr, 1, nullptr, nullptr, 0, 0,
                                nullptr, nullptr, 32, nullptr, 0, 64, nullptr));
  EXPECT_ERR(ic_gemv_w8a8(nullptr, 17, 128, 128, nullptr, 8, 128, nullptr, nullptr, nullptr, 0, nullptr, 0, 8,
                          nullptr));
  EXPECT_ERR(ic_unpack_int4_to_int8(nullptr, 4, 64, 16, nullptr, 64, nullptr));
  EXPECT_ERR(ic_unpack_int4_to_float(nullptr, nullptr, 3, 4, 64, 32, nullptr, 2, 64, nullptr));
  EXPECT_ERR(ic_gemm_w4a8_acc_i32(nullptr, 4, 100, 100, nullptr, 4, 50, nullptr, 3, nullptr, 0, nullptr));
  // the e3m2 path
  EXPECT_ERR(ic_f6_split_activations(nullptr, 16, 192, 192, nullptr, nullptr));
  EXPECT_ERR(ic_f6_repack_weights(nullptr, 16, 256, 64, nullptr, nullptr));
  EXPECT_ERR(ic_gemm_w4a8_f6(nullptr, 16, 256, nullptr, 16, nullptr, 1, nullptr, nullptr, 0, nullptr, 0, 16,
                             nullptr));
  EXPECT_ERR(ic_gemm_w4a8_f6(nullptr, 16, 256, nullptr, 12, nullptr, 2, nullptr, nullptr, 0, nullptr, 0, 12,
                             nullptr));
  expect(ic_f6_activation_bytes(17, 256) == 2 * 2 * 3072, "ic_f6_activation_bytes");
  expect(ic_f6_weight_bytes(17, 256) == 2 * 2 * 1536, "ic_f6_weight_bytes");
  expect(ic_f6_activation_bytes(16, 200) == 0, "ic_f6_activation_bytes K");
  // no-alloc: plans beyond the scratch are refused before any launch
  EXPECT_ERR(ic_gemm_w4a8_noalloc(nullptr, 512, 65536, 65536, nullptr, 3072, 32768, nullptr, 512, nullptr, nullptr,
                                  0, nullptr, IC_DTYPE_BF16, 3072, nullptr));
  // M = 0 is a no-op that touches nothing
  EXPECT_OK(ic_gemm_w8a8(nullptr, 0, 128, 128, nullptr, 64, 128, nullptr, nullptr, nullptr, 0, nullptr, 0, 64,
                         nullptr));
  // split-K planning (pure host logic) over a range of shapes
  for (long long M = 17; M <= 4096; M *= 3)
    for (long long N = 64; N <= 16384; N *= 4)
      for (long long K = 128; K <= 16384; K *= 2) {
        const int64_t b1 = ic_gemm_splitk_bytes(M, N, K, 1, 0), b2 = ic_gemm_splitk_bytes(M, N, K, K / 128, 1);
        expect(b1 >= 0 && b2 >= 0, "ic_gemm_splitk_bytes");
      }
  if (failures) {
    std::fprintf(stderr, "%d failures\n", failures);
    return 1;
  }
  std::puts("ABI sanitizer driver: clean");
  return 0;
}
