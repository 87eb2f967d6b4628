// Fast-path prep + quantize kernels for f16 activations with a LayerNorm or
// RMSNorm of each row first (ic_norm_rotate_quantize): SmoothRot factors and
// perm read at run time here; rows with both go to rq_norm_f16_both.hip.
#include "rq_fast.h"

hipError_t ic_rq_norm_f16(const ic_rotq_args& a, hipStream_t st) {
  if (a.sr_rcp != nullptr && a.perm != nullptr) return ic_rq_norm_f16_both(a, st);
  if (a.norm == IC_NORM_LAYER) return launch_fast<IC_DTYPE_F16, kRqGeneral, IC_NORM_LAYER>(a, st);
  return launch_fast<IC_DTYPE_F16, kRqGeneral, IC_NORM_RMS>(a, st);
}
