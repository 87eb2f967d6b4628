/* Exercises the C oracle (oracle/intcrush_oracle.c) under AddressSanitizer
 * and UndefinedBehaviorSanitizer (tests/test_sanitizers.py builds and runs
 * it): every entry point on odd shapes, pads, perms, all dtypes, both
 * Hadamard forms, grouped and per-row epilogues, with a few invariants
 * checked on the way.  Exit status 0 = clean. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

double oc_round(double d, int dtype);
int oc_prepare(const float* x, int dtype, int64_t M, int64_t K_in, const float* srf, int R, int64_t K_w,
               const int32_t* perm, const float* smf, float* out, int64_t* n_inexact, int fast);
void oc_quantize(const float* x, int64_t M, int64_t K, int8_t* q, float* s);
void oc_quantize_rne(const float* x, int64_t M, int64_t K, int8_t* q, float* s);
void oc_unpack_int4(const uint8_t* packed, int64_t N, int64_t K, int64_t ldp, int8_t* out);
void oc_pack_int4(const int8_t* vals, int64_t N, int64_t K, uint8_t* out);
void oc_dequant_w4a16(const uint8_t* packed, const float* s_w, int64_t G, int64_t N, int64_t K, int64_t ldp,
                      int dtype, float* out);
int64_t oc_gemm_acc(const int8_t* A, int64_t M, int64_t K, const int8_t* W, int64_t N, int64_t G, int32_t* acc);
void oc_epilogue(const int32_t* acc, int64_t M, int64_t N, int64_t G, const float* s_a, const float* s_w,
                 const float* bias, int out_dtype, float* out);

static uint32_t rng = 12345u;
static float frand(void) {
  rng = rng * 1664525u + 1013904223u;
  return ((float)(rng >> 8) / 16777216.0f) * 2.0f - 1.0f;
}
#define CHECK(c)                                              \
  do {                                                        \
    if (!(c)) {                                               \
      fprintf(stderr, "check failed at line %d: %s\n", __LINE__, #c); \
      return 1;                                               \
    }                                                         \
  } while (0)

int main(void) {
  /* pack / unpack round trip, odd K */
  for (int K = 1; K <= 33; K += 8) {
    const int N = 3, Kp = (K + 1) / 2;
    int8_t* v = malloc(N * K);
    uint8_t* p = malloc(N * Kp);
    int8_t* u = malloc(N * K);
    for (int i = 0; i < N * K; ++i) v[i] = (int8_t)((i * 7) % 16 - 8);
    oc_pack_int4(v, N, K, p);
    oc_unpack_int4(p, N, K, Kp, u);
    for (int i = 0; i < N * K; ++i) CHECK(u[i] == v[i]);
    float* w = malloc(sizeof(float) * N * K);
    float sw[3 * 2] = {1e-3f, 2e-3f, 3e-3f, 4e-3f, 5e-3f, 6e-3f};
    oc_dequant_w4a16(p, sw, K % 2 == 0 && K >= 2 ? 2 : 1, N, K, Kp, 0, w);
    free(v); free(p); free(u); free(w);
  }
  /* prepare: every rot size, dtypes, pads, perm, SmoothRot, old-smooth, both forms */
  const int Rs[6] = {0, 16, 64, 256, 1024, 4096};
  for (int dt = 0; dt < 3; ++dt)
    for (int ri = 0; ri < 6; ++ri)
      for (int fast = 0; fast < 2; ++fast) {
        const int R = Rs[ri], M = 3;
        if (R >= 1024 && !fast) continue; /* the direct sum is quadratic in R */
        const int64_t K_in = R ? R + R / 2 + 3 : 77;
        const int64_t K_r = R ? (K_in + R - 1) / R * R : K_in;
        const int64_t K_w = K_r + 16;
        float* x = malloc(sizeof(float) * M * K_in);
        float* srf = malloc(sizeof(float) * K_in);
        float* smf = malloc(sizeof(float) * K_w);
        int32_t* perm = malloc(sizeof(int32_t) * K_w);
        float* out = malloc(sizeof(float) * M * K_w);
        for (int64_t i = 0; i < M * K_in; ++i) x[i] = (float)oc_round(frand() * 4.0f, dt);
        x[0] = 1e-30f;
        for (int64_t i = 0; i < K_in; ++i) srf[i] = (float)oc_round(1.0 + 0.5 * fabs(frand()), dt);
        for (int64_t i = 0; i < K_w; ++i) {
          smf[i] = (float)oc_round(1.0 + 0.25 * fabs(frand()), dt);
          perm[i] = (int32_t)((i * 7 + 3) % K_w);
        }
        int64_t inexact = 0;
        CHECK(oc_prepare(x, dt, M, K_in, srf, R, K_w, perm, smf, out, &inexact, fast) == 0);
        CHECK(oc_prepare(x, dt, M, K_in, NULL, R, K_w, NULL, NULL, out, &inexact, fast) == 0);
        for (int64_t i = K_r; i < K_w; ++i) CHECK(out[i] == 0.0f); /* the pad after the rotated width */
        int8_t* q = malloc(M * K_w);
        float s[3];
        oc_quantize(out, M, K_w, q, s);
        oc_quantize_rne(out, M, K_w, q, s);
        for (int m = 0; m < M; ++m) CHECK(s[m] > 0.0f);
        free(x); free(srf); free(smf); free(perm); free(out); free(q);
      }
  /* bad arguments are refused */
  {
    float x[32] = {0}, out[64];
    CHECK(oc_prepare(x, 0, 1, 32, NULL, 32, 32, NULL, NULL, out, NULL, 1) != 0);  /* not a power of 4 */
    CHECK(oc_prepare(x, 0, 1, 32, NULL, 16, 16, NULL, NULL, out, NULL, 1) != 0);  /* K_w below the rotated width */
  }
  /* GEMM accumulators and epilogues, per-row and grouped, with and without bias */
  {
    const int M = 5, N = 7, K = 384;
    int8_t* A = malloc(M * K);
    int8_t* W = malloc(N * K);
    for (int i = 0; i < M * K; ++i) A[i] = (int8_t)(i % 255 - 127);
    for (int i = 0; i < N * K; ++i) W[i] = (int8_t)((i * 3) % 16 - 8);
    for (int G = 1; G <= 3; G += 2) {
      int32_t* acc = malloc(sizeof(int32_t) * G * M * N);
      CHECK(oc_gemm_acc(A, M, K, W, N, G, acc) == 0);
      float sa[5], sw[7 * 3], bias[7], out[5 * 7];
      for (int i = 0; i < M; ++i) sa[i] = 1e-3f * (i + 1);
      for (int i = 0; i < N * G; ++i) sw[i] = 2e-3f * (i + 1);
      for (int i = 0; i < N; ++i) bias[i] = 0.5f * i;
      for (int dt = 0; dt < 3; ++dt) {
        oc_epilogue(acc, M, N, G, sa, sw, bias, dt, out);
        oc_epilogue(acc, M, N, G, sa, sw, NULL, dt, out);
      }
      free(acc);
    }
    free(A); free(W);
  }
  puts("oracle sanitizer driver: clean");
  return 0;
}
