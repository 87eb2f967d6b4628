// The INT8 / packed-INT4 MFMA GEMMs with the activation / residual epilogue
// compiled in (a separate translation unit: its instantiations double the
// kernel set, and this way they compile in parallel with the plain ones).
#include "gemm_i8.h"

int ic_gemm_run_epi(const ic_gemm::GemmArgs& g, hipStream_t st, const char* who, bool force_generic) {
  return run_gemm_t<true>(g, st, who, force_generic);
}
