// ic_int4_interleave_k: packed INT4 rows from the checkpoint's nibble order
// (byte b: k = 2b low, 2b + 1 high; _quant_utils.py:67-80) to the
// K-interleaved order the W4A8 kernels expand without byte permutes (byte
// 4d + j: k = 8d + j low, 8d + 4 + j high).  A permutation of the nibbles
// inside each 4-byte word, run once per layer and device.
#include "ic_common.h"

namespace {

// One thread per 4-byte word (8 weights) of a row; byte loads and stores, so
// rows may have any stride and alignment, and out may be w itself (each
// thread reads its word before writing it).
__global__ __launch_bounds__(256) void int4_interleave_kernel(const uint8_t* w, int64_t ldw, uint8_t* out,
                                                              int64_t ldo, int64_t N, int64_t words) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= N * words) return;
  const int64_t n = i / words, d = i - n * words;
  const uint8_t* src = w + n * ldw + 4 * d;
  uint32_t p = 0;
#pragma unroll
  for (int b = 0; b < 4; ++b) p |= (uint32_t)src[b] << (8 * b);
  uint32_t q = 0;  // nibble k of p (weight k of the word) to its K-interleaved place
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    q |= ((p >> (4 * j)) & 15u) << (8 * j);
    q |= ((p >> (16 + 4 * j)) & 15u) << (8 * j + 4);
  }
  uint8_t* dst = out + n * ldo + 4 * d;
#pragma unroll
  for (int b = 0; b < 4; ++b) dst[b] = (uint8_t)(q >> (8 * b));
}

}  // namespace

extern "C" int ic_int4_interleave_k(const uint8_t* w_packed, int64_t N, int64_t K, int64_t ldw, uint8_t* w_kil,
                                    int64_t ldo, void* stream) {
  const char* who = "ic_int4_interleave_k";
  if (N < 0 || K <= 0 || K % 8 != 0 || ldw < K / 2 || ldo < K / 2)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: K=%lld must be a positive multiple of 8, row strides >= K/2", who,
                        (long long)K);
  const bool overlap = (const uint8_t*)w_kil < w_packed + N * ldw && w_packed < w_kil + N * ldo;
  if (overlap && !(w_kil == w_packed && ldo == ldw))
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: output overlaps the input other than in place", who);
  if (N == 0) return IC_OK;
  if (!w_packed || !w_kil) return ic_set_error(IC_ERR_INVALID_ARG, "%s: null pointer", who);
  const int64_t words = K / 8, total = N * words;
  int4_interleave_kernel<<<dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream>>>(
      w_packed, ldw, w_kil, ldo, N, words);
  return ic_check_launch(who);
}
