// INT4 -> 16-bit weight dequantization with packed math, shared by the W4A16
// GEMM and GEMV kernels: w = RN_dt(q * RN_dt(s)) for 8 weights at a time.
#pragma once
#include "ic_common.h"

namespace {

typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef float v2f __attribute__((ext_vector_type(2)));

// Per-column dequantization constants: f16 keeps the pair
// (RN_f16(s), RN_f16(s)); bf16 keeps sb = RN_bf16(s) and -8 * sb (exact).
struct DeqScale {
  uint32_t s2;    // f16: two copies of RN_f16(s)
  float sb, m8s;  // bf16
};
template <int DT> IC_DEV DeqScale deq_scale(float s) {
  DeqScale d;
  if constexpr (DT == IC_DTYPE_F16) {
    const uint32_t h = __builtin_bit_cast(u16, (_Float16)s);
    d.s2 = h | (h << 16);
    d.sb = d.m8s = 0.0f;
  } else {
    d.s2 = 0;
    d.sb = bf16_to_f32(f32_to_bf16(s));
    d.m8s = -8.0f * d.sb;
  }
  return d;
}

// Dequantize 8 INT4 values (one packed dword, low nibble = even k) to 8 16-bit
// values of type DT in natural k order (4 dwords, two values each).
//   u = q + 8 in [0, 15] is the nibble with its sign bit flipped.
//   f16:  the halves 0x6400 | u are the f16 numbers 1024 + u; subtracting 1032
//         gives q exactly, and one f16 multiply by RN_f16(s) rounds q*s once.
//   bf16: u as f32, fma(u, sb, -8*sb) = q*sb exactly (12 significant bits),
//         then one RN-even conversion to bf16.
template <int DT> IC_DEV void deq8(uint32_t P, const DeqScale& d, uint32_t* o) {
  const uint32_t t = (P & 0x0f0f0f0fu) ^ 0x08080808u;         // u of k = 0, 2, 4, 6
  const uint32_t h = ((P >> 4) & 0x0f0f0f0fu) ^ 0x08080808u;  // u of k = 1, 3, 5, 7
  const uint32_t e = __builtin_amdgcn_perm(h, t, 0x05010400u);  // u0 u1 u2 u3
  const uint32_t f = __builtin_amdgcn_perm(h, t, 0x07030602u);  // u4 u5 u6 u7
  if constexpr (DT == IC_DTYPE_F16) {
    const uint32_t c64 = 0x64646464u;
    const uint32_t w[4] = {__builtin_amdgcn_perm(c64, e, 0x04010400u), __builtin_amdgcn_perm(c64, e, 0x04030402u),
                           __builtin_amdgcn_perm(c64, f, 0x04010400u), __builtin_amdgcn_perm(c64, f, 0x04030402u)};
    const v2h sc = __builtin_bit_cast(v2h, d.s2);
    const v2h off = {(_Float16)1032.0f, (_Float16)1032.0f};
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(v2h, w[i]) - off) * sc);
  } else {
    const uint32_t u[2] = {e, f};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float a = __builtin_fmaf((float)((u[i] >> (16 * j)) & 0xffu), d.sb, d.m8s);
        const float b = __builtin_fmaf((float)((u[i] >> (16 * j + 8)) & 0xffu), d.sb, d.m8s);
        o[2 * i + j] = __builtin_bit_cast(uint32_t, __builtin_convertvector((v2f){a, b}, v2bf));
      }
    }
  }
}

}  // namespace
