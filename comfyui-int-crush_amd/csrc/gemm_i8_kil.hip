// gemm_i8_big_kernel on packed INT4 in the K-interleaved nibble order (every
// INT4 weight mode, both 16-bit outputs, with and without the activation /
// residual epilogue).  A translation unit of its own so that these
// instantiations compile in parallel with gemm_i8.hip and gemm_i8_epi.hip.
#include <type_traits>

#include "gemm_i8.h"

hipError_t ic_launch_big_kil(const ic_gemm::GemmArgs& g, int out_dt, bool epi, int mode, hipStream_t st) {
  auto go = [&](auto o, auto e) -> hipError_t {
    constexpr int O = decltype(o)::value;
    constexpr bool E = decltype(e)::value;
    switch (mode) {
      case big::G128: return launch_big<O, E, big::G128, true>(g, st);
      case big::G64: return launch_big<O, E, big::G64, true>(g, st);
      case big::G32: return launch_big<O, E, big::G32, true>(g, st);
      case big::ROW4: return launch_big<O, E, big::ROW4, true>(g, st);
    }
    return hipErrorInvalidValue;
  };
  using F16 = std::integral_constant<int, IC_DTYPE_F16>;
  using BF16 = std::integral_constant<int, IC_DTYPE_BF16>;
  if (out_dt == IC_DTYPE_F16) return epi ? go(F16{}, std::true_type{}) : go(F16{}, std::false_type{});
  if (out_dt == IC_DTYPE_BF16) return epi ? go(BF16{}, std::true_type{}) : go(BF16{}, std::false_type{});
  return hipErrorInvalidValue;
}
