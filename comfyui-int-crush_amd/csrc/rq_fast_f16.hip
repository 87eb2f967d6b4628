// Fast-path prep + quantize kernels for f16 activations with either SmoothRot
// factors or a perm (run-time flags); rows with neither go to the plain
// instantiations (rq_fast_f16_plain.hip), rows with both to rq_fast_f16_both.hip.
#include "rq_fast.h"

hipError_t ic_rq_fast_f16(const ic_rotq_args& a, hipStream_t st) {
  if (a.sr_rcp == nullptr && a.perm == nullptr) return ic_rq_fast_f16_plain(a, st);
  if (a.sr_rcp != nullptr && a.perm != nullptr) return ic_rq_fast_f16_both(a, st);
  return launch_fast<IC_DTYPE_F16, kRqGeneral>(a, st);
}
