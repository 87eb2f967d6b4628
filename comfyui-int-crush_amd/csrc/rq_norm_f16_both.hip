// Fast-path prep + quantize kernels for f16 activations with a LayerNorm or
// RMSNorm of each row first and both SmoothRot factors and a perm.
#include "rq_fast.h"

hipError_t ic_rq_norm_f16_both(const ic_rotq_args& a, hipStream_t st) {
  if (a.norm == IC_NORM_LAYER) return launch_fast<IC_DTYPE_F16, kRqBoth, IC_NORM_LAYER>(a, st);
  return launch_fast<IC_DTYPE_F16, kRqBoth, IC_NORM_RMS>(a, st);
}
