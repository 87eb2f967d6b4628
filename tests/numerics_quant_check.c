/* Exhaustive check of the f32 quantize formula of the fast prep kernels
 * (quant_code_mk in comfyui-int-crush_amd/csrc/ic_common.h) against the
 * reference rule (kernels/triton_quantize.py:133-146):
 *
 *   s = max(m, 1e-8) / 127 (f32),  code = trunc(RN32(RN32(v / s) +- 0.5))
 *
 * for every value m >= 0 of a 16-bit type (the row abs-max after rounding to
 * that type) and every value v of that type with |v| <= m, both signs.
 * Prints the mismatch counts of the kernel formula (must be 0) and of the
 * single-rounding shortcut trunc(RN32(v * RN32(1/s) +- 0.5)) (nonzero: the
 * check can see a wrong formula).
 *
 * usage: numerics_quant_check <0 = fp16 | 1 = bf16>
 * Built with -ffp-contract=off: every a * b + c below is rounded twice unless
 * written as fmaf, exactly as the GPU code is compiled and written.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float from_f16(uint16_t h) {
  const int e = (h >> 10) & 31, m = h & 1023;
  float v;
  if (e == 0) v = ldexpf((float)m, -24);
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = ldexpf((float)(m | 1024), e - 25);
  return (h >> 15) ? -v : v;
}

static float from_bf16(uint16_t h) {
  const uint32_t w = (uint32_t)h << 16;
  float f;
  memcpy(&f, &w, 4);
  return f;
}

static int reference_code(float v, float s) {
  const float q = v / s;
  const float r = q >= 0.0f ? q + 0.5f : q - 0.5f;
  int c = (int)r;
  return c < -128 ? -128 : (c > 127 ? 127 : c);
}

static int kernel_code(float v, float s, float r) {
  const float q0 = fmaf(v, r, 0.0f); /* RN32(v r); a zero product becomes +0 */
  const float e = fmaf(-q0, s, v);
  const float q = fmaf(e, r, q0);
  return (int)(q + copysignf(0.5f, q));
}

static int shortcut_code(float v, float r) {
  const float q = v * r;
  return (int)(q + copysignf(0.5f, q));
}

int main(int argc, char** argv) {
  if (argc != 2) return 2;
  const int bf = atoi(argv[1]);
  const int top = bf ? 0x7f7f : 0x7bff; /* largest finite positive bit pattern */
  long long pairs = 0, bad = 0, bad_shortcut = 0;
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : pairs, bad, bad_shortcut)
  for (int mh = 0; mh <= top; ++mh) {
    const float m = bf ? from_bf16((uint16_t)mh) : from_f16((uint16_t)mh);
    const float s = fmaxf(m, 1e-8f) / 127.0f;
    const float r = 1.0f / s;
    for (int vh = 0; vh <= mh; ++vh) {
      const float a = bf ? from_bf16((uint16_t)vh) : from_f16((uint16_t)vh);
      for (int sign = 0; sign < 2; ++sign) {
        const float v = sign ? -a : a;
        const int want = reference_code(v, s);
        pairs += 1;
        bad += kernel_code(v, s, r) != want;
        bad_shortcut += shortcut_code(v, r) != want;
      }
    }
  }
  printf("pairs %lld mismatches %lld shortcut_mismatches %lld\n", pairs, bad, bad_shortcut);
  return 0;
}
