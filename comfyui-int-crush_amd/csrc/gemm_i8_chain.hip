// Chained MLP epilogue entry points: the up-projection GEMM (W8A8 or W4A8)
// with its activation, whose tiles are then prepared in LDS as the next
// linear's activation (SmoothRot divide + R-block Hadamard) before they are
// stored.  Kernels in gemm_i8.h (ROT instantiations of gemm_i8_kernel).
#include "gemm_i8.h"

namespace {

int log4_of(int r) {
  switch (r) {
    case 16: return 2;
    case 64: return 3;
    case 256: return 4;
    default: return -1;
  }
}

int run_chain(GemmArgs g, int rot_size, hipStream_t st, const char* who) {
  if (g.M < 0 || g.N <= 0 || g.K <= 0 || g.lda < g.K || g.ldc < g.N)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: bad shape M=%d N=%d K=%d lda=%lld ldc=%lld", who, g.M, g.N, g.K,
                        (long long)g.lda, (long long)g.ldc);
  if (g.int4 ? (g.ldb * 2 < g.K) : (g.ldb < g.K))
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: weight row stride %lld too small for K=%d", who, (long long)g.ldb,
                        g.K);
  if (g.out_dt != IC_DTYPE_F16 && g.out_dt != IC_DTYPE_BF16)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: the chained output is the next linear's activation: f16 or bf16",
                        who);
  if (g.bias && g.bias_dt != IC_DTYPE_F16 && g.bias_dt != IC_DTYPE_BF16 && g.bias_dt != IC_DTYPE_F32)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: bias dtype must be f16/bf16/f32", who);
  if (g.epi.act < 0 || g.epi.act > 3)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: activation must be 0 (none), 1 (SiLU), 2 (GELU) or 3 (GELU tanh)",
                        who);
  if ((g.epi.sr_rcp == nullptr) != (g.epi.sr_f == nullptr))
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: SmoothRot reciprocals and factors come together", who);
  const int log4r = log4_of(rot_size);
  if (log4r < 0)
    return ic_set_error(IC_ERR_UNSUPPORTED, "%s: rot_size %d: the chained epilogue rotates blocks of 16, 64 or 256 "
                        "columns inside its 256-column tiles", who, rot_size);
  if (g.N % rot_size != 0)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: N=%d is not a multiple of rot_size %d", who, g.N, rot_size);
  if (g.G < 1 || (g.G > 1 && (g.K % g.G != 0 || (g.K / g.G) % kBK != 0)))
    return ic_set_error(IC_ERR_UNSUPPORTED, "%s: num_groups %d: group sizes must be multiples of 128", who, g.G);
  // the tile kernel's operand rules and its staged (16-byte row) output path
  if (g.K % kBK != 0 || ((uintptr_t)g.A & 15) || ((uintptr_t)g.B & 15) || (g.lda & 15) || (g.ldb & 15) ||
      ((uintptr_t)g.C & 15) || (g.ldc & 7) || g.ldc >= (1LL << 24) || !dma_strides_ok(g))
    return ic_set_error(IC_ERR_UNSUPPORTED, "%s: K a multiple of 128, 16-byte aligned operands, row strides and "
                        "output, output row stride a multiple of 8 elements (and row strides below 2^31 / 320 "
                        "bytes) are required", who);
  if (g.M == 0) return IC_OK;
  if (!g.A || !g.B || !g.s_a || !g.s_w || !g.C) return ic_set_error(IC_ERR_INVALID_ARG, "%s: null pointer argument", who);
  hipError_t e;
  if (!g.int4) e = launch_chain<Tile<128, 256, 2, 3, false, 0>>(g, log4r, st);
  else if (g.G > 1) e = launch_chain<Tile<128, 256, 2, 3, true, 128>>(g, log4r, st);
  else e = launch_chain<Tile<128, 256, 2, 3, true, 0>>(g, log4r, st);
  if (e != hipSuccess) return ic_set_error(IC_ERR_LAUNCH, "%s: %s", who, hipGetErrorString(e));
  return IC_OK;
}

}  // namespace

extern "C" {

int ic_gemm_w8a8_chain(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const int8_t* w, int64_t N, int64_t ldw,
                       const float* s_a, const float* s_w, const void* bias, int bias_dtype, int activation,
                       const float* sr_rcp, const float* sr_f, int rot_size, void* out, int out_dtype, int64_t ldo,
                       void* stream) {
  ic_epi epi{activation, nullptr, 0, 0};
  epi.sr_rcp = sr_rcp;
  epi.sr_f = sr_f;
  GemmArgs g{xq, ldx, (const uint8_t*)w, ldw, s_a, s_w, 1, bias, bias_dtype, out, out_dtype, ldo,
             (int)M, (int)N, (int)K, nullptr, false, nullptr, 0, epi};
  return run_chain(g, rot_size, (hipStream_t)stream, "ic_gemm_w8a8_chain");
}

int ic_gemm_w4a8_chain(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const uint8_t* w_packed, int64_t N,
                       int64_t ldw, const float* s_w, int64_t num_groups, const float* s_a, const void* bias,
                       int bias_dtype, int activation, const float* sr_rcp, const float* sr_f, int rot_size,
                       void* out, int out_dtype, int64_t ldo, void* stream) {
  ic_epi epi{activation, nullptr, 0, 0};
  epi.sr_rcp = sr_rcp;
  epi.sr_f = sr_f;
  GemmArgs g{xq, ldx, w_packed, ldw, s_a, s_w, (int)num_groups, bias, bias_dtype, out, out_dtype, ldo,
             (int)M, (int)N, (int)K, nullptr, true, nullptr, 0, epi};
  return run_chain(g, rot_size, (hipStream_t)stream, "ic_gemm_w4a8_chain");
}

}  // extern "C"
