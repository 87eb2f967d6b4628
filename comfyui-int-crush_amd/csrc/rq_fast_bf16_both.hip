// Fast-path prep + quantize kernels for bf16 activations with both SmoothRot
// factors and a perm (the PermuQuant + SmoothRot checkpoints).
#include "rq_fast.h"

hipError_t ic_rq_fast_bf16_both(const ic_rotq_args& a, hipStream_t st) {
  return launch_fast<IC_DTYPE_BF16, kRqBoth>(a, st);
}
