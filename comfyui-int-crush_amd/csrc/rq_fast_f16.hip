// Fast-path prep + quantize kernels for f16 activations.
#include "rq_fast.h"

hipError_t ic_rq_fast_f16(const ic_rotq_args& a, hipStream_t st) { return launch_fast<IC_DTYPE_F16>(a, st); }
