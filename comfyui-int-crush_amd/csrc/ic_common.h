// Shared device helpers for the INT-Crush gfx950 kernels.
//
// Numeric conventions (all kernels):
//   * dtype codes follow include/intcrush.h: 0 = fp16, 1 = bf16, 2 = fp32.
//   * Every float conversion is IEEE round-to-nearest-even.  The library is
//     built with -ffp-contract=off so that a*b+c is never silently fused;
//     fused multiply-adds are written explicitly where the algorithm wants them.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/intcrush.h"

#define IC_DEV __device__ __forceinline__

// ---------------------------------------------------------------- host side
// Thread-local error message + launch checking (defined in capi.cpp).
int ic_set_error(int code, const char* fmt, ...);
int ic_check_launch(const char* who);
int ic_num_cus();  // compute units of the current device
// hipFuncSetAttribute(MaxDynamicSharedMemorySize) once per kernel and device;
// done points at the caller's 64 per-device flags.
hipError_t ic_set_lds_limit(const void* kern, int bytes, unsigned char* done);
// Validation of the epilogue arguments (activation code, residual dtype and
// stride) shared by the entry points that take them (gemm_i8.hip).
int ic_check_epi(const char* who, int activation, const void* residual, int residual_dtype, int64_t ldr, int64_t N);
// GEMV routing tests shared by the GEMM entry points (gemv.hip); strides in
// bytes.  The W4A8 GEMV takes per-row scales and groups of multiples of 32
// columns whose fold sums fit its LDS.
bool ic_gemv_applicable(int64_t M, int64_t K, const void* x, int64_t ldx_bytes, const void* w, int64_t ldw_bytes);
bool ic_gemv_w4a8_groups_ok(int64_t M, int64_t K, int64_t num_groups);

// Arguments of the fused preparation kernels (internal; the ABI is flat).
struct ic_rotq_args {
  const void* x; int dtype; int64_t M, K_in, ldx;
  const float* sr_rcp; const float* sr_f; int rot_size; int64_t K_w;
  const int32_t* perm; const float* sm_rcp; const float* sm_f;
  int8_t* q_out; int64_t ldq; float* s_out;
  void* y_out; int64_t ldy;
  // row normalisation applied first (ic_norm_rotate_quantize): kind
  // IC_NORM_LAYER / IC_NORM_RMS, optional f32 [K_in] scale and shift, eps
  int norm = 0; const float* nw = nullptr; const float* nb = nullptr; float eps = 0.0f;
};

typedef uint16_t u16;
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- 16-bit floats
IC_DEV float f16_to_f32(u16 h) { return (float)__builtin_bit_cast(_Float16, h); }
IC_DEV u16 f32_to_f16(float f) { return __builtin_bit_cast(u16, (_Float16)f); }
IC_DEV float bf16_to_f32(u16 b) { return __uint_as_float((uint32_t)b << 16); }
// Round-to-nearest-even f32 -> bf16 with the gfx950 conversion instruction
// (one VALU op; NaN stays a quiet NaN).
IC_DEV u16 f32_to_bf16(float f) { return __builtin_bit_cast(u16, (__bf16)f); }

template <int DT> IC_DEV float ld_as_f32(const void* p, int64_t i) {
  if constexpr (DT == IC_DTYPE_F16) return f16_to_f32(((const u16*)p)[i]);
  else if constexpr (DT == IC_DTYPE_BF16) return bf16_to_f32(((const u16*)p)[i]);
  else return ((const float*)p)[i];
}
IC_DEV float ld_any_f32(const void* p, int dt, int64_t i) {
  if (dt == IC_DTYPE_F16) return f16_to_f32(((const u16*)p)[i]);
  if (dt == IC_DTYPE_BF16) return bf16_to_f32(((const u16*)p)[i]);
  return ((const float*)p)[i];
}
template <int DT> IC_DEV void st_from_f32(void* p, int64_t i, float v) {
  if constexpr (DT == IC_DTYPE_F16) ((u16*)p)[i] = f32_to_f16(v);
  else if constexpr (DT == IC_DTYPE_BF16) ((u16*)p)[i] = f32_to_bf16(v);
  else ((float*)p)[i] = v;
}

// Round an f32 to the 16-bit activation type and back (RN-even), f32 passes through.
template <int DT> IC_DEV float round_to_dt(float v) {
  if constexpr (DT == IC_DTYPE_F16) return f16_to_f32(f32_to_f16(v));
  else if constexpr (DT == IC_DTYPE_BF16) return bf16_to_f32(f32_to_bf16(v));
  else return v;
}

// Smallest positive normal of the activation type: below it the type is
// subnormal and the reciprocal-multiply shortcut of the divide is not exact.
template <int DT> IC_DEV constexpr float dt_min_normal() {
  if constexpr (DT == IC_DTYPE_F16) return 6.103515625e-05f;  // 2^-14
  else return 1.1754943508222875e-38f;                        // 2^-126
}

// Correctly rounded RN_dt(x / f) for x, f values of type DT, given
// rcp = RN32(1/f) and f itself (read only on the slow path).
// Fast path: RN_dt(RN32(x*rcp)).  Exhaustive CPU checks over every finite
// (x, f) fp16 and bf16 pair show the fast path equals the exactly rounded
// quotient unless the product is non-finite or nonzero below the normal range
// of DT; those lanes take the IEEE f32 divide (RN32 then RN_dt is innocuous
// for a quotient of two values with <= 11 significant bits).
template <int DT> IC_DEV float div_round_dt(float x, float rcp, const float* fptr, int64_t k) {
  if constexpr (DT == IC_DTYPE_F32) {
    return x / fptr[k];  // f32 activations: the reference divides in f32 directly
  } else {
    float p = x * rcp;
    float ap = __builtin_fabsf(p);
    bool fast = (ap >= dt_min_normal<DT>() && ap <= 3.4028234663852886e38f) || p == 0.0f;
    if (__builtin_expect(fast, 1)) return round_to_dt<DT>(p);
    return round_to_dt<DT>(x / fptr[k]);
  }
}

// ------------------------------------------------------------ fp64 -> 16-bit
// Round-to-odd to 24 significant bits: truncate the 29 low mantissa bits of an
// fp64 and set the kept LSB if any dropped bit was set.  The result is exactly
// representable in f32, and RN_dt(rto24(y)) == RN_dt(y) for any 16-bit type
// (24 >= p + 2 with p <= 11), which is the classic round-to-odd argument.
IC_DEV float rto24(double y) {
  uint64_t b = (uint64_t)__double_as_longlong(y);
  uint32_t lo = (uint32_t)b;
  uint32_t hi = (uint32_t)(b >> 32);
  uint32_t sticky = (lo & 0x1fffffffu) ? 1u : 0u;
  lo = (lo & 0xe0000000u) | (sticky << 29);
  return (float)__longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// RN of an fp64 value to DT, returned as the f32 holding that exact value.
template <int DT> IC_DEV float round_f64_to_dt(double y) {
  if constexpr (DT == IC_DTYPE_F32) return (float)y;
  else return round_to_dt<DT>(rto24(y));
}

// ------------------------------------------------------------ quantization
// Reference rule (triton_quantize.py:133-146): s = max(m, 1e-8)/127 in f32;
// q = trunc(RN32(RN32(v/s) +- 0.5)) clamped to [-128, 127].  v/s is formed as
// RN32(v * RN64(1/s)) in fp64, which equals the IEEE f32 quotient for every v
// with <= 24 significant bits and normal s (the quotient is never an f32
// midpoint and lies >= 2^-48 relative from one; the fp64 error is < 2^-52).
IC_DEV float quant_scale(float m) { return __builtin_fmaxf(m, 1e-8f) / 127.0f; }
IC_DEV int quant_code(float v, double rs) {
  float q = (float)((double)v * rs);
  float r = q >= 0.0f ? q + 0.5f : q - 0.5f;
  int c = (int)r;  // v_cvt_i32_f32 truncates toward zero (saturating)
  c = c < -128 ? -128 : c;
  c = c > 127 ? 127 : c;
  return c;
}

// The same code for 16-bit activations v with |v| <= m (the row abs-max the
// scale was built from), without the clamp and in f32 arithmetic.  No clamp:
// |RN32(v/s)| <= RN32(127 * (1 + 2^-24)) < 127.5, so trunc(q +- 0.5) already
// lies in [-127, 127]; infinite or NaN quotients only arise with m = inf or
// v = NaN, where v_cvt_i32_f32 returns 0 and the clamped form returns 0 too.
// The quotient: with r = RN32(1/s), it is corrected once (Markstein):
//   q0 = RN32(v r),  e = RN32(v - s q0) (exact),  q = RN32(q0 + e r)
// and q = RN32(v/s) for every fp16 / bf16 value v with |v| <= m, m itself a
// value of that type (the row abs-max after rounding): checked exhaustively
// over all such pairs (v, m) of both types and both signs, every code equal
// to the reference rule (tests/numerics_quant_check.c); a single rounding of
// v r (+- 0.5) is not (thousands of pairs per type differ).  v = +-inf or NaN gives 0 as the fp64 form does.
IC_DEV int quant_code_mk(float v, float s, float r) {
  // q0 = RN32(v r), as an FMA with a +0 addend: for a 16-bit v widened from
  // fp16 the compiler then reads v in its fp16 form (v_fma_mix_f32) and needs
  // no conversion.  Only a zero product can change (-0 becomes +0), and it
  // gives code 0 either way.
  const float q0 = __builtin_fmaf(v, r, 0.0f);
  const float e = __builtin_fmaf(-q0, s, v);
  const float q = __builtin_fmaf(e, r, q0);
  return (int)(q + __builtin_copysignf(0.5f, q));
}

// Low bytes of four ints packed little-endian into one dword.
IC_DEV uint32_t pack4_lo_bytes(int c0, int c1, int c2, int c3) {
  const uint32_t lo = __builtin_amdgcn_perm((uint32_t)c1, (uint32_t)c0, 0x0c0c0400u);
  const uint32_t hi = __builtin_amdgcn_perm((uint32_t)c3, (uint32_t)c2, 0x04000c0cu);
  return lo | hi;
}

// ------------------------------------------------------------ packed INT4
// Packed INT4 weight rows come in two nibble orders (two's complement nibbles
// either way):
//   plain (the checkpoint format, _quant_utils.py:67-80): byte b holds
//     k = 2b in its low nibble and k = 2b + 1 in its high nibble;
//   K-interleaved (ic_int4_interleave_k): byte 4d + j holds k = 8d + j in its
//     low nibble and k = 8d + 4 + j in its high nibble (j = 0..3).
// A dword of 8 nibbles expands to 8 int8 values 16*q in natural k order from
// two masked copies, lo = the low nibbles moved up, hi = the high nibbles in
// place (bytes 16*q, exactly; the factor 16 is removed in the epilogues).
// The plain order then needs two byte permutes; the K-interleaved one takes
// lo and hi as they are.  W4Sel holds the permutes' selectors, so that
// kernels keeping them serve either order with the same instructions.
struct W4Sel {
  uint32_t s0, s1;
};
constexpr W4Sel kW4Plain{0x05010400u, 0x07030602u};  // q0 q1 q2 q3 | q4 q5 q6 q7 from (hi, lo)
constexpr W4Sel kW4Kil{0x03020100u, 0x07060504u};    // lo | hi
IC_DEV void unpack8_x16(uint32_t P, uint32_t& w0, uint32_t& w1, W4Sel sel = kW4Plain) {
  const uint32_t lo = (P << 4) & 0xf0f0f0f0u;
  const uint32_t hi = P & 0xf0f0f0f0u;
  w0 = __builtin_amdgcn_perm(hi, lo, sel.s0);
  w1 = __builtin_amdgcn_perm(hi, lo, sel.s1);
}
IC_DEV void unpack8_x16_kil(uint32_t P, uint32_t& w0, uint32_t& w1) {
  w0 = (P << 4) & 0xf0f0f0f0u;
  w1 = P & 0xf0f0f0f0u;
}
// Nibble index (byte * 2 + high) of weight k in a packed row.
IC_DEV int w4_nibble_index(int k, bool kil) {
  return kil ? ((k & ~7) + 2 * (k & 3) + ((k >> 2) & 1)) : k;
}

// ------------------------------------------------------------ reductions
IC_DEV float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = __builtin_fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Maximum over the wave of a value that is >= +0 and never NaN (an abs-max
// built with fmaxf), returned in every lane.  Such floats order as their bit
// patterns, so the reduction runs on integers through DPP lane moves within
// each row of 16 lanes, then the four row results are read as scalars.
IC_DEV float wave_max_nonneg(float v) {
  int x = __float_as_int(v);
  x = max(x, __builtin_amdgcn_mov_dpp(x, 0xB1, 0xf, 0xf, false));   // quad_perm [1,0,3,2]
  x = max(x, __builtin_amdgcn_mov_dpp(x, 0x4E, 0xf, 0xf, false));   // quad_perm [2,3,0,1]
  x = max(x, __builtin_amdgcn_mov_dpp(x, 0x141, 0xf, 0xf, false));  // row_half_mirror
  x = max(x, __builtin_amdgcn_mov_dpp(x, 0x140, 0xf, 0xf, false));  // row_mirror
  const int r01 = max(__builtin_amdgcn_readlane(x, 0), __builtin_amdgcn_readlane(x, 16));
  const int r23 = max(__builtin_amdgcn_readlane(x, 32), __builtin_amdgcn_readlane(x, 48));
  return __int_as_float(max(r01, r23));
}

// ------------------------------------------------------------ GEMM epilogue options
// After the dequant and bias of the INT8 GEMMs (kernels/triton_int8_gemm.py:119-130):
// an activation on the f32 value, then a residual [M, N] (f16/bf16/f32, row
// stride ldr) added, then the rounding to the output dtype.
//   act 0: none; 1: SiLU v * sigmoid(v); 2: GELU 0.5 v (1 + erf(v / sqrt 2));
//   3: GELU with the tanh approximation (not in the reference; the MLPs of
//   DiT models such as Flux use it).
struct ic_epi {
  int act = 0;
  const void* res = nullptr;
  int res_dt = 0;
  int64_t ldr = 0;
  // chained MLP epilogue (ic_gemm_*_chain): the next linear's SmoothRot
  // reciprocals RN32(1/f) and factors f, per output column (both NULL: none)
  const float* sr_rcp = nullptr;
  const float* sr_f = nullptr;
};

// v * sigmoid(t) = v / (1 + e^-t) from the hardware exp2 and reciprocal
// (e^-t as 2^(-t log2 e); both instructions are within 1 ulp, the argument's
// rounding adds |t| 2^-24 relative to e^-t, a sigmoid error of at most
// 0.25 |t| 2^-24 after the derivative).  e^-t overflowing to +inf gives
// v * 0; underflowing to 0 gives v.
IC_DEV float mul_sigmoid(float v, float t) {
  const float e = __builtin_amdgcn_exp2f(t * -1.44269504088896341f);
  return v * __builtin_amdgcn_rcpf(1.0f + e);
}

// GELU 0.5 v (1 + erf(v / sqrt 2)) with erf from Abramowitz & Stegun,
// Handbook of Mathematical Functions, eq. 7.1.26: for a >= 0,
// 1 - erf(a) = P(t) e^(-a^2), t = 1 / (1 + p a), |error| <= 1.5e-7.  The
// tail 1 + erf(-a) is that product itself (no cancellation), 1 + erf(a) is
// 2 minus it.  In f32 with the hardware exp2 / reciprocal the result stays
// within 2^-21.7 (|v| + |GELU(v)|) of the exact value (checked against
// float64 erf on a dense grid, each instruction perturbed by +-1 ulp).
IC_DEV float gelu_erf(float v) {
  const float a = fabsf(v) * 0.70710678118654752f;
  const float t = __builtin_amdgcn_rcpf(1.0f + 0.3275911f * a);
  const float p =
      t * (0.254829592f + t * (-0.284496736f + t * (1.421413741f + t * (-1.453152027f + t * 1.061405429f))));
  const float q = p * __builtin_amdgcn_exp2f((a * a) * -1.44269504088896341f);  // 1 - erf(a)
  return (v * 0.5f) * (v >= 0.0f ? 2.0f - q : q);
}

IC_DEV float epi_act(float v, int act) {
  if (act == 1) {
    v = mul_sigmoid(v, v);  // SiLU
  } else if (act == 2) {
    v = gelu_erf(v);
  } else if (act == 3) {
    // 0.5 v (1 + tanh(u)) = v sigmoid(2u), u = sqrt(2/pi) (v + 0.044715 v^3)
    const float u2 = 1.5957691216057308f * (v + 0.044715f * (v * v * v));
    v = mul_sigmoid(v, u2);
  }
  return v;
}

IC_DEV float epi_apply(float v, const ic_epi& e, int m, int n) {
  v = epi_act(v, e.act);
  if (e.res != nullptr) v = v + ld_any_f32(e.res, e.res_dt, (int64_t)m * e.ldr + n);
  return v;
}

// GEMV bodies with an epilogue (gemv.hip), used by the GEMM entry points for M <= 16.
int ic_gemv_w8a8_epi(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const int8_t* w, int64_t N, int64_t ldw,
                     const float* s_a, const float* s_w, const void* bias, int bias_dtype, void* out, int out_dtype,
                     int64_t ldo, const ic_epi& epi, void* stream);
int ic_gemv_w4a8_epi(const int8_t* xq, int64_t M, int64_t K, int64_t ldx, const uint8_t* w_packed, int64_t N,
                     int64_t ldw, const float* s_w, int64_t num_groups, const float* s_a, const void* bias,
                     int bias_dtype, void* out, int out_dtype, int64_t ldo, const ic_epi& epi, void* stream,
                     W4Sel sel = kW4Plain);
