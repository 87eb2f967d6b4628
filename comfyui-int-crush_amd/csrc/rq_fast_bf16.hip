// Fast-path prep + quantize kernels for bf16 activations with SmoothRot
// factors and/or a perm (run-time flags); rows without either go to the
// PLAIN instantiations in rq_fast_bf16_plain.hip.
#include "rq_fast.h"

hipError_t ic_rq_fast_bf16(const ic_rotq_args& a, hipStream_t st) {
  if (a.sr_rcp == nullptr && a.perm == nullptr) return ic_rq_fast_bf16_plain(a, st);
  return launch_fast<IC_DTYPE_BF16, false>(a, st);
}
