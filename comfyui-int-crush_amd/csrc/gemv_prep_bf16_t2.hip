// Single-launch prep + GEMV kernels for bf16 activations, rows of at most
// 8192 positions (one source file per set, compiled in parallel).
#include "gemv_prep.h"

hipError_t ic_prep_gemv_bf16_t2(const gemvp::PrepGemvLaunch& L, hipStream_t st) {
  return gemvp::launch_prep_gemv<IC_DTYPE_BF16, 2>(L, st);
}
