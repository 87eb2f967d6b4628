// Single-launch prep + GEMV kernels for f16 activations, rows of at most
// 4096 positions (one source file per set, compiled in parallel).
#include "gemv_prep.h"

hipError_t ic_prep_gemv_f16_t1(const gemvp::PrepGemvLaunch& L, hipStream_t st) {
  return gemvp::launch_prep_gemv<IC_DTYPE_F16, 1>(L, st);
}
