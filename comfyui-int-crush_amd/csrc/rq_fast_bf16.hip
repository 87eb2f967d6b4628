// Fast-path prep + quantize kernels for bf16 activations.
#include "rq_fast.h"

hipError_t ic_rq_fast_bf16(const ic_rotq_args& a, hipStream_t st) { return launch_fast<IC_DTYPE_BF16>(a, st); }
