// Fast-path prep + quantize kernels for f16 activations without SmoothRot
// factors or perm (rotation, pad and quantization only).
#include "rq_fast.h"

hipError_t ic_rq_fast_f16_plain(const ic_rotq_args& a, hipStream_t st) {
  return launch_fast<IC_DTYPE_F16, kRqPlain>(a, st);
}
