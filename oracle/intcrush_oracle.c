/*
 * intcrush_oracle.c - CPU restatement of the INT-Crush quantized-linear forward.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the GPU kernels are
 * compared against; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  It is never part of the product path.
 *
 * Each function restates the reference semantics (ThunderFun/ComfyUI-INT-Crush,
 * file:line cited per function) with plain IEEE double/float arithmetic.  The
 * algorithms are deliberately written differently from the GPU kernels
 * (closed-form Hadamard entries instead of butterflies, IEEE f32 division
 * instead of reciprocal tricks, scalar loops instead of MFMA tiles) so that a
 * shared mistake is unlikely.
 *
 * dtype codes: 0 = fp16, 1 = bf16, 2 = fp32.  Activation values are passed as
 * f32 arrays holding exact values of the dtype.
 *
 * Build: gcc -O2 -fPIC -shared -ffp-contract=off (see oracle/Makefile).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ rounding */
/* Exact round-to-nearest-even of a double to a binary format with p
 * significand bits, minimum normal exponent emin and largest finite maxv.
 * The division by a power of two and nearbyint are exact, so this is a single
 * correct rounding of the double's value. */
static double rnd_format(double d, int p, int emin, double maxv) {
  if (d == 0.0 || isnan(d) || isinf(d)) return d;
  int e;
  frexp(d, &e);
  int E = e - 1;
  if (E < emin) E = emin;
  double q = ldexp(1.0, E - (p - 1));
  double r = nearbyint(d / q) * q;
  if (fabs(r) > maxv) return copysign(INFINITY, d);
  if (r == 0.0) return copysign(0.0, d);
  return r;
}

double oc_round(double d, int dtype) {
  switch (dtype) {
    case 0: return rnd_format(d, 11, -14, 65504.0);
    case 1: return rnd_format(d, 8, -126, 3.3895313892515355e38);
    default: return (double)(float)d; /* x86-64 SSE cvtsd2ss: RN-even */
  }
}

/* fp16 / bf16 bit patterns of exact values (for fixtures). */
uint16_t oc_f16_bits(double v) {
  v = oc_round(v, 0);
  uint16_t s = signbit(v) ? 0x8000 : 0;
  double a = fabs(v);
  if (isnan(v)) return 0x7e00;
  if (isinf(a)) return s | 0x7c00;
  if (a == 0.0) return s;
  int e;
  frexp(a, &e);
  int E = e - 1;
  if (E < -14) return s | (uint16_t)(a * 16777216.0); /* subnormal: multiple of 2^-24 */
  uint16_t m = (uint16_t)(ldexp(a, 10 - E) - 1024.0);
  return s | (uint16_t)((E + 15) << 10) | m;
}

/* ------------------------------------------------------------------ prep */
/* Regular Hadamard entry: H = (H4/2)^{(x)k} with H4 = [[1,1,1,-1],[1,1,-1,1],
 * [1,-1,1,1],[-1,1,1,1]] (_quant_utils.py:67-93).  H4[a][b] = -1 iff a+b == 3,
 * so H[i][j] = 2^-k * (-1)^{#digits d with i_d + j_d == 3}. */
static double had_entry(int i, int j, int k) {
  int neg = 0;
  for (int d = 0; d < k; ++d) {
    int a = (i >> (2 * d)) & 3, b = (j >> (2 * d)) & 3;
    if (a + b == 3) neg ^= 1;
  }
  return ldexp(neg ? -1.0 : 1.0, -k);
}

/* Whether the double sum of a block is provably exact: all terms are
 * multiples of 2^qmin and every partial sum is below R * 2^(emax+1); that
 * fits in 53 bits when (emax + 1 + log2 R) - qmin <= 53. */
static int block_sum_exact(const double* v, int R, int p) {
  int emax = -10000, qmin = 10000, lr = 0;
  while ((1 << lr) < R) ++lr;
  for (int j = 0; j < R; ++j) {
    if (v[j] == 0.0) continue;
    int e;
    frexp(v[j], &e);
    if (e - 1 > emax) emax = e - 1;
    if (e - p < qmin) qmin = e - p; /* quantum of a p-bit significand */
  }
  if (emax == -10000) return 1;
  return (emax + 1 + lr) - qmin <= 53;
}

/* Per-digit evaluation of y = H x for one block: for each base-4 digit d,
 * y[..a..] = sum_b (H4[a][b] / 2) x[..b..].  Equal to the direct sum whenever
 * block_sum_exact holds (every partial is then exact in double). */
static void had_fast(double* v, int R, int k) {
  static const double H4[4][4] = {{1, 1, 1, -1}, {1, 1, -1, 1}, {1, -1, 1, 1}, {-1, 1, 1, 1}};
  for (int d = 0; d < k; ++d) {
    int st = 1 << (2 * d);
    for (int base = 0; base < R; ++base) {
      if ((base >> (2 * d)) & 3) continue;
      double in[4], o[4];
      for (int b = 0; b < 4; ++b) in[b] = v[base + b * st];
      for (int a = 0; a < 4; ++a) {
        o[a] = 0.0;
        for (int b = 0; b < 4; ++b) o[a] += H4[a][b] * 0.5 * in[b];
      }
      for (int a = 0; a < 4; ++a) v[base + a * st] = o[a];
    }
  }
}

/*
 * bf16 rows: inputs more than 43 - 2k binades below the largest magnitude of
 * their Hadamard block (R = 4^k) are replaced by zero before the rotation,
 * |x| < 2^(e_max - (43 - 2k)) with e_max = floor(log2 max|x|) over the
 * block's finite values.  The remaining inputs span at most 43 - 2k binades,
 * so every butterfly partial sum is exact in double (block_sum_exact holds);
 * the flushed values change an output by less than 2^-(43 - 3k) of the
 * block's largest input.  fp16 and f32 rows are not flushed.
 */
static void flush_small_bf16(double* v, int R, int k) {
  double mx = 0.0;
  for (int j = 0; j < R; ++j) {
    const double a = fabs(v[j]);
    if (isfinite(a) && a > mx) mx = a;
  }
  if (mx == 0.0) return;
  int e;
  frexp(mx, &e);
  const double thr = ldexp(1.0, (e - 1) - (43 - 2 * k));
  for (int j = 0; j < R; ++j)
    if (fabs(v[j]) < thr) v[j] = 0.0;
}

/*
 * _prep_activation (_ops.py:337-365) + old SmoothQuant (_ops.py:529-533) for
 * one row block [M, K_in] -> [M, K_w]:
 *   x / RN_dt(f)  rounded to dt                       (_ops.py:349-350)
 *   pad to a multiple of R, y = x_blk @ H^T rounded to dt (_quant_utils.py:127-147)
 *   pad to K_w (_ops.py:355-358); y = y[..., perm]    (_ops.py:360-363)
 *   y / RN_dt(smooth) rounded to dt                    (_ops.py:529-533)
 * srf / smf are the dtype-rounded factors (NULL = absent).  The Hadamard is
 * evaluated as a direct sum of closed-form entries in double (fast = 0) or
 * digit by digit (fast = 1); blocks whose sum is not provably exact are
 * reported in *n_inexact (never for fp16 inputs).
 * Returns 0, or -1 on bad arguments.
 */
int oc_prepare(const float* x, int dtype, int64_t M, int64_t K_in, const float* srf, int R,
               int64_t K_w, const int32_t* perm, const float* smf, float* out, int64_t* n_inexact,
               int fast) {
  int k = 0;
  if (R != 0) {
    int r = R;
    while (r > 1) {
      if (r & 3) return -1;
      r >>= 2;
      ++k;
    }
    if (k < 1) return -1;
  }
  const int64_t K_r = R ? ((K_in + R - 1) / R) * R : K_in;
  if (K_w < K_r) return -1;
  const int p = dtype == 0 ? 11 : dtype == 1 ? 8 : 24;
  double* a = (double*)calloc((size_t)K_r, sizeof(double));
  double* y = (double*)calloc((size_t)K_w, sizeof(double));
  if (!a || !y) {
    free(a);
    free(y);
    return -1;
  }
  int64_t inexact = 0;
  for (int64_t m = 0; m < M; ++m) {
    const float* xr = x + m * K_in;
    for (int64_t j = 0; j < K_r; ++j) {
      double v = j < K_in ? (double)xr[j] : 0.0;
      if (srf && j < K_in) v = oc_round(v / (double)srf[j], dtype);
      a[j] = v;
    }
    for (int64_t j = 0; j < K_w; ++j) y[j] = 0.0;
    if (R == 0) {
      for (int64_t j = 0; j < K_r; ++j) y[j] = a[j];
    } else {
      for (int64_t b0 = 0; b0 < K_r; b0 += R) {
        if (dtype == 1) flush_small_bf16(a + b0, R, k);
        if (!block_sum_exact(a + b0, R, p)) ++inexact;
        if (fast) {
          had_fast(a + b0, R, k);
          for (int i = 0; i < R; ++i) y[b0 + i] = oc_round(a[b0 + i], dtype);
        } else {
          for (int i = 0; i < R; ++i) {
            double s = 0.0;
            for (int j = 0; j < R; ++j) s += had_entry(i, j, k) * a[b0 + j];
            y[b0 + i] = oc_round(s, dtype);
          }
        }
      }
    }
    float* orow = out + m * K_w;
    for (int64_t j = 0; j < K_w; ++j) {
      double v = perm ? y[perm[j]] : y[j];
      if (smf) v = oc_round(v / (double)smf[j], dtype);
      orow[j] = (float)v;
    }
  }
  free(a);
  free(y);
  if (n_inexact) *n_inexact = inexact;
  return 0;
}

/*
 * Per-token dynamic INT8 quantization, GPU rule of kernels/triton_quantize.py:109-146:
 *   m = max_k |x|;  s = max(m, 1e-8) / 127  (f32);
 *   q = trunc(f32(x/s) +- 0.5) clamped to [-128, 127].
 * Division and addition are IEEE f32 (x86-64 SSE, no contraction).
 */
void oc_quantize(const float* x, int64_t M, int64_t K, int8_t* q, float* s) {
  for (int64_t m = 0; m < M; ++m) {
    const float* xr = x + m * K;
    float mx = 0.0f;
    for (int64_t j = 0; j < K; ++j) {
      float a = fabsf(xr[j]);
      if (a > mx) mx = a;
    }
    volatile float floor_ = 1e-8f;
    float sc = (mx > floor_ ? mx : floor_) / 127.0f;
    s[m] = sc;
    for (int64_t j = 0; j < K; ++j) {
      volatile float qf = xr[j] / sc;
      volatile float r = qf >= 0.0f ? qf + 0.5f : qf - 0.5f;
      long c = (long)r; /* truncation toward zero */
      if (c < -128) c = -128;
      if (c > 127) c = 127;
      q[m * K + j] = (int8_t)c;
    }
  }
}

/* torch.round (half-to-even) variant used by the reference CPU fallback,
 * kernels/triton_quantize.py:43-54. */
void oc_quantize_rne(const float* x, int64_t M, int64_t K, int8_t* q, float* s) {
  for (int64_t m = 0; m < M; ++m) {
    const float* xr = x + m * K;
    float mx = 0.0f;
    for (int64_t j = 0; j < K; ++j) {
      float a = fabsf(xr[j]);
      if (a > mx) mx = a;
    }
    float sc = (mx > 1e-8f ? mx : 1e-8f) / 127.0f;
    s[m] = sc;
    for (int64_t j = 0; j < K; ++j) {
      volatile float qf = xr[j] / sc;
      double c = nearbyint((double)qf);
      if (c < -128) c = -128;
      if (c > 127) c = 127;
      q[m * K + j] = (int8_t)c;
    }
  }
}

/* ------------------------------------------------------------------ weights */
/* INT4 unpack, _quant_utils.py:185-197: low nibble = even k, two's complement. */
void oc_unpack_int4(const uint8_t* packed, int64_t N, int64_t K, int64_t ldp, int8_t* out) {
  for (int64_t n = 0; n < N; ++n)
    for (int64_t k = 0; k < K; ++k) {
      int b = packed[n * ldp + k / 2];
      int v = (k & 1) ? (b >> 4) & 15 : b & 15;
      out[n * K + k] = (int8_t)(v >= 8 ? v - 16 : v);
    }
}

/* INT4 pack, _quant_utils.py:170-182 (odd K zero-padded). */
void oc_pack_int4(const int8_t* vals, int64_t N, int64_t K, uint8_t* out) {
  int64_t kp = (K + 1) / 2;
  for (int64_t n = 0; n < N; ++n)
    for (int64_t j = 0; j < kp; ++j) {
      int lo = vals[n * K + 2 * j];
      int hi = 2 * j + 1 < K ? vals[n * K + 2 * j + 1] : 0;
      out[n * kp + j] = (uint8_t)(((lo < 0 ? lo + 16 : lo) & 15) | (((hi < 0 ? hi + 16 : hi) & 15) << 4));
    }
}

/* W4A16 dequantized weight, kernels/triton_int4_unpack.py:49-56 generalised to
 * [N, G] group scales (_quant_utils.py:237-270): w = RN_dt(q * RN_dt(s[n, k/gs])). */
void oc_dequant_w4a16(const uint8_t* packed, const float* s_w, int64_t G, int64_t N, int64_t K,
                      int64_t ldp, int dtype, float* out) {
  const int64_t gs = K / G;
  for (int64_t n = 0; n < N; ++n)
    for (int64_t k = 0; k < K; ++k) {
      int b = packed[n * ldp + k / 2];
      int v = (k & 1) ? (b >> 4) & 15 : b & 15;
      int q = v >= 8 ? v - 16 : v;
      double s = oc_round((double)s_w[n * G + k / gs], dtype);
      out[n * K + k] = (float)oc_round((double)q * s, dtype);
    }
}

/* ------------------------------------------------------------------ GEMM */
/* Integer stage of triton_int8_gemm.py:96-103 / triton_w4a8_gemm.py:84-91:
 * acc[g][m][n] = sum_{k in group g} a[m,k] * w[n,k], exact (int64, then
 * checked to fit int32).  G = 1 gives the plain accumulator.  Returns the
 * number of accumulators that overflowed int32. */
int64_t oc_gemm_acc(const int8_t* A, int64_t M, int64_t K, const int8_t* W, int64_t N, int64_t G,
                    int32_t* acc) {
  const int64_t gs = K / G;
  int64_t ovf = 0;
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n)
      for (int64_t g = 0; g < G; ++g) {
        int64_t s = 0;
        const int8_t* a = A + m * K + g * gs;
        const int8_t* w = W + n * K + g * gs;
        for (int64_t k = 0; k < gs; ++k) s += (int64_t)a[k] * (int64_t)w[k];
        if (s > INT32_MAX || s < INT32_MIN) ++ovf;
        acc[(g * M + m) * N + n] = (int32_t)s;
      }
  return ovf;
}

/* Dequant epilogue.
 *   G == 1 (triton_int8_gemm.py:105-117): v = f32(acc) * (s_a[m] * s_w[n]) + bias[n]
 *   G  > 1 (group layout of _quant_utils.py:237-270): f = fma chain over g of
 *          f32(acc_g) * s_w[n,g]; v = f * s_a[m] + bias[n]
 * All f32 with no contraction except the explicit fmaf; bias holds the
 * bias values as f32 (NULL = none); out = RN_dt(v) held as f32. */
void oc_epilogue(const int32_t* acc, int64_t M, int64_t N, int64_t G, const float* s_a,
                 const float* s_w, const float* bias, int out_dtype, float* out) {
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      volatile float v;
      if (G == 1) {
        volatile float sc = s_a[m] * s_w[n];
        v = (float)acc[m * N + n] * sc;
      } else {
        float f = 0.0f;
        for (int64_t g = 0; g < G; ++g) f = fmaf((float)acc[(g * M + m) * N + n], s_w[n * G + g], f);
        v = f * s_a[m];
      }
      if (bias) v = v + bias[n];
      out[m * N + n] = (float)oc_round((double)v, out_dtype);
    }
}
