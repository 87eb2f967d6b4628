// Device helpers shared by the fused prep + quantize kernels (generic path in
// rotate_quant.hip, fast path in rq_fast.h).
#pragma once
#include "ic_common.h"

namespace rq {

constexpr int kThreads = 256;
constexpr int kTile = 4096;       // positions per tile (kThreads * 16)
constexpr int kMaxTiles = 4;      // K_w <= 16384 for the fused single-pass kernel
constexpr int kPadStride = 18;    // 16 doubles + 2 pad per 16-position row of the transpose buffer

IC_DEV void h4(double& a, double& b, double& c, double& d) {
  double s = (a + b) + (c + d);
  double ya = __builtin_fma(s, 0.5, -d);
  double yb = __builtin_fma(s, 0.5, -c);
  double yc = __builtin_fma(s, 0.5, -b);
  double yd = __builtin_fma(s, 0.5, -a);
  a = ya; b = yb; c = yc; d = yd;
}
// radix-4 stage on the low / high 2-bit digit of a 16-element register array
IC_DEV void stage_lo(double* v) {
#pragma unroll
  for (int a = 0; a < 4; ++a) h4(v[4 * a + 0], v[4 * a + 1], v[4 * a + 2], v[4 * a + 3]);
}
IC_DEV void stage_hi(double* v) {
#pragma unroll
  for (int a = 0; a < 4; ++a) h4(v[a], v[4 + a], v[8 + a], v[12 + a]);
}
// physical slot of logical position p in the padded transpose buffer
IC_DEV int tslot(int p) { return p + 2 * (p >> 4); }

template <int DT> IC_DEV u16 f32_bits16(float v) {
  if constexpr (DT == IC_DTYPE_F16) return f32_to_f16(v);
  else return f32_to_bf16(v);
}
// Two f32 values rounded to DT (RN-even) in one packed conversion
// (v_cvt_pk_f16_f32 / v_cvt_pk_bf16_f32), a in the low half.
template <int DT> IC_DEV uint32_t pack2_bits16(float a, float b) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  if constexpr (DT == IC_DTYPE_F16) {
    typedef _Float16 h16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, h16x2));
  } else {
    typedef __bf16 b16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, b16x2));
  }
}
template <int DT> IC_DEV float bits16_f32(u16 b) {
  if constexpr (DT == IC_DTYPE_F16) return f16_to_f32(b);
  else return bf16_to_f32(b);
}

// Load 16 consecutive values starting at element p0 (zero past n) as f32.
// Whole in-bounds 16-element runs use 16-byte loads when the base is aligned.
template <int DT> IC_DEV void load16(const void* base, int p0, int n, bool vec_ok, float* out) {
  constexpr int ESZ = DT == IC_DTYPE_F32 ? 4 : 2;
  if (vec_ok && p0 + 16 <= n && ((((uintptr_t)base) & 15) == 0)) {
    const v4u* src = (const v4u*)((const char*)base + (int64_t)p0 * ESZ);
    if constexpr (ESZ == 2) {
      v4u a = src[0], b = src[1];
      uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        out[2 * i] = bits16_f32<DT>((u16)(w[i] & 0xffffu));
        out[2 * i + 1] = bits16_f32<DT>((u16)(w[i] >> 16));
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v4u a = src[i];
        out[4 * i] = __uint_as_float(a.x);
        out[4 * i + 1] = __uint_as_float(a.y);
        out[4 * i + 2] = __uint_as_float(a.z);
        out[4 * i + 3] = __uint_as_float(a.w);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j) out[j] = (p0 + j < n) ? ld_as_f32<DT>(base, p0 + j) : 0.0f;
  }
}
IC_DEV void load16i(const int32_t* base, int p0, int n, int* out) {
  if (p0 + 16 <= n && ((((uintptr_t)base) & 15) == 0)) {
    const v4u* src = (const v4u*)(base + p0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v4u a = src[i];
      out[4 * i] = (int)a.x; out[4 * i + 1] = (int)a.y; out[4 * i + 2] = (int)a.z; out[4 * i + 3] = (int)a.w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j) out[j] = (p0 + j < n) ? base[p0 + j] : 0;
  }
}

// Layout of register element j of thread t after the rotation phases for rot
// size class RC (0: none/16, 1: 64/256, 2: 1024/4096, 3: 1024 rotated inside
// each wave's own 1024 positions), tile-local position.
template <int RC> IC_DEV int tile_pos(int t, int j) {
  if constexpr (RC == 0) return 16 * t + j;
  else if constexpr (RC == 1) return 256 * (t >> 4) + 16 * j + (t & 15);
  else if constexpr (RC == 2) return 256 * j + t;
  else return 1024 * (t >> 6) + 256 * (j & 3) + 4 * (t & 63) + (j >> 2);
}

// LDS layouts of the fast path and the chained GEMM epilogue (doubles in the
// exchange buffer, 16-bit values in the row buffer).  Exchange slot of tile
// position p: 2 doubles of padding per 16 positions and 16 per 256.  Then the
// b128 row writes of 16 lanes hit 16 distinct 4-bank groups (row stride 36
// dwords) and the transposed b64 reads of the four 16-lane groups of a wave
// land on alternate halves of the 64 banks.  Row-buffer address of position
// p: 16 values of padding per 256, so the strided writes of the four 16-lane
// groups of a wave use distinct banks.
IC_DEV int xslot(int p) { return p + 2 * (p >> 4) + 16 * (p >> 8); }
template <int TILE> constexpr int xbuf_doubles() { return TILE + 2 * (TILE / 16) + 16 * (TILE / 256); }
// The same buffer without the 16 per 256 (tslot): the fast path's R = 64 /
// 256 exchange keeps its transposed reads on alternate bank halves instead by
// letting the odd 16-lane groups read their 16 rows in the order h ^ 8.
template <int TILE> constexpr int tslot_doubles() { return TILE + 2 * (TILE / 16); }
IC_DEV int rbaddr(int p) { return p + 16 * (p >> 8); }
template <int NT, int TILE> constexpr int rowbuf_len() { return NT * TILE + 16 * (NT * TILE / 256); }

// RN_dt(y) of an fp64 value through RN32: exact unless RN32(y) is itself a
// rounding boundary of DT (a midpoint between neighbours, including the
// overflow threshold) or lies below DT's normal range.  Boundary test on the
// f32 bits: the bits below DT's precision are exactly 100...0.
template <int DT> IC_DEV uint32_t rn32_boundary_key(float z) {
  const uint32_t w = __float_as_uint(z);
  if constexpr (DT == IC_DTYPE_F16) return (w ^ 0x1000u) & 0x1fffu;  // zero iff (w & 0x1fff) == 0x1000
  else return (w ^ 0x8000u) & 0xffffu;
}

constexpr int kFastMaxTiles = 4;  // fast path: K_w <= 16384

// ---- bf16 flush of values far below their Hadamard block's maximum.
// The fp64 butterflies are exact when the nonzero inputs of a block (8-bit
// significands) span at most kFlushSpan(k) = 43 - 2k binades (R = 4^k): each
// partial sum is then an integer multiple of the smallest input's quantum
// below 2^53.  bf16 rows can span far more (GELU outputs reach 1e-37 next to
// values of 100); values more than kFlushSpan(k) binades below the block's
// largest magnitude, |x| < 2^(e_max - kFlushSpan(k)), are replaced by zero
// before the rotation, which then stays exact.  Such a value moves an output
// by at most 2^-(kFlushSpan(k) - k) of the block's largest input, below what
// the reference's own fp32-accumulating matmul (_quant_utils.py:117-147)
// resolves; the oracle applies the same rule.  fp16 rows (40 binades of
// range) are always exact and never flushed.
template <int LOG4R> constexpr int kFlushSpan() { return 43 - 2 * LOG4R; }

// Per-run statistics the bf16 flush rule needs, over a thread's 16 values:
// the largest |x| as bits (integer maximum of the bits without the sign, so
// NaN > inf > any finite value) and the smallest |x| (f32 minimum, which
// ignores NaN; zero when the run holds a zero).  Callers that already form
// them while rounding the run pass them in.
struct Bf16RunStats {
  uint32_t amax_bits;
  float amin;
};
IC_DEV Bf16RunStats bf16_run_stats(const float* xs) {
  Bf16RunStats st{0u, __builtin_huge_valf()};
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const uint32_t a = __float_as_uint(xs[j]) & 0x7fffffffu;
    st.amax_bits = st.amax_bits > a ? st.amax_bits : a;
    st.amin = __builtin_fminf(st.amin, __builtin_fabsf(xs[j]));
  }
  return st;
}

// Maximum / minimum of an unsigned value over aligned groups of G lanes (G a
// power of 4 up to 64), in every lane of the group: DPP moves inside rows of
// 16 lanes (quad permutations, then the half-row and row mirrors), lane
// shuffles across rows.
template <int G, bool MAX> IC_DEV uint32_t group_reduce_u32(uint32_t v) {
  auto op = [](uint32_t a, uint32_t b) { return MAX ? (a > b ? a : b) : (a < b ? a : b); };
  auto dpp = [](uint32_t x, int ctrl) -> uint32_t {
    switch (ctrl) {
      case 0: return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0xB1, 0xf, 0xf, false);   // quad_perm [1,0,3,2]
      case 1: return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x4E, 0xf, 0xf, false);   // quad_perm [2,3,0,1]
      case 2: return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x141, 0xf, 0xf, false);  // row_half_mirror
      default: return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x140, 0xf, 0xf, false); // row_mirror
    }
  };
  if constexpr (G >= 4) {
    v = op(v, dpp(v, 0));
    v = op(v, dpp(v, 1));
  }
  if constexpr (G >= 16) {
    v = op(v, dpp(v, 2));
    v = op(v, dpp(v, 3));
  }
  if constexpr (G >= 64) {
    v = op(v, (uint32_t)__shfl_xor((int)v, 16, 64));
    v = op(v, (uint32_t)__shfl_xor((int)v, 32, 64));
  }
  return v;
}

// xs: the 16 consecutive input positions of this thread (after the SmoothRot
// divide); a block of R positions is the R/16 consecutive threads of one
// aligned group (R = 4096: the four waves of the workgroup, reduced through
// xred, 2 * TH / 64 words of LDS, with one workgroup barrier).  e_max is the
// f32 exponent field of the block's largest |x|; bf16 subnormals have field 0.
// The smallest nonzero |x| is the run's smallest |x| unless the run holds a
// zero, when it is searched for.
template <int LOG4R, int TH>
IC_DEV void bf16_flush_small(float* xs, uint32_t* xred, Bf16RunStats st) {
  constexpr int G = (1 << (2 * LOG4R)) / 16;  // threads per block
  uint32_t mx = st.amax_bits;                 // max |x| bits
  uint32_t mn;                                // min nonzero |x| bits - 1 (none: 0xffffffff)
  if (st.amin > 0.0f) {
    mn = __float_as_uint(st.amin) - 1u;
  } else {
    mn = 0xffffffffu;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint32_t am1 = (__float_as_uint(xs[j]) & 0x7fffffffu) - 1u;  // zero wraps to the maximum
      mn = mn < am1 ? mn : am1;
    }
  }
  mx = group_reduce_u32<(G < 64 ? G : 64), true>(mx);
  mn = group_reduce_u32<(G < 64 ? G : 64), false>(mn);
  if constexpr (G > 64) {
    static_assert(G == TH, "a block of more than one wave spans the whole workgroup");
    if ((threadIdx.x & 63) == 0) {
      xred[2 * (threadIdx.x >> 6)] = mx;
      xred[2 * (threadIdx.x >> 6) + 1] = mn;
    }
    __syncthreads();
#pragma unroll
    for (int w = 0; w < TH / 64; ++w) {
      mx = mx > xred[2 * w] ? mx : xred[2 * w];
      mn = mn < xred[2 * w + 1] ? mn : xred[2 * w + 1];
    }
  }
  const int emax = (int)(mx >> 23), emin = (int)((mn + 1u) >> 23);
  const bool wide = mn != 0xffffffffu && emax - emin > kFlushSpan<LOG4R>();
  if (__builtin_expect(__any(wide), 0)) {  // wave-uniform
    const uint32_t thr = emax > kFlushSpan<LOG4R>() ? (uint32_t)(emax - kFlushSpan<LOG4R>()) << 23 : 0u;
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if ((__float_as_uint(xs[j]) & 0x7fffffffu) < thr) xs[j] = 0.0f;
  }
}
template <int LOG4R, int TH>
IC_DEV void bf16_flush_small(float* xs, uint32_t* xred) {
  bf16_flush_small<LOG4R, TH>(xs, xred, bf16_run_stats(xs));
}

// Global -> LDS DMA of 16 bytes per lane (global_load_lds_dwordx4): lane i
// reads base + voff and writes LDS address lds + 16 * i.  base and lds must
// be wave-uniform (they are read into scalar registers here).  Issued from
// inline assembly so that the compiler does not track it; its completion is
// waited for explicitly with wait_vm_n.  The memory clobber keeps the
// compiler's own memory accesses on their side of the issue.
IC_DEV void dma16_lds(uint32_t voff, const void* base, uint32_t lds) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  const void* sb = (const void*)(uintptr_t)(((uint64_t)hi << 32) | lo);
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(__builtin_amdgcn_readfirstlane(lds)),
               "v"(voff), "s"(sb)
               : "m0", "memory");
}

// Block until at most n vector-memory operations of this wave are in flight
// (they retire in issue order); n is wave-uniform, 0..4.
template <int N> IC_DEV void wait_vm_imm() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }
IC_DEV void wait_vm_n(int n) {
  if (n <= 0) wait_vm_imm<0>();
  else if (n == 1) wait_vm_imm<1>();
  else if (n == 2) wait_vm_imm<2>();
  else if (n == 3) wait_vm_imm<3>();
  else wait_vm_imm<4>();
}

// Instantiation sets of the fast-path kernels (see rq_fast.h).
constexpr int kRqPlain = 0;    // no SmoothRot factors, no perm
constexpr int kRqGeneral = 1;  // either one; flags read at run time
constexpr int kRqBoth = 2;     // both

}  // namespace rq

// Fast-path launchers (rq_fast_f16.hip / rq_fast_bf16.hip); argument checks
// and fast_path_ok() are done by the caller.
hipError_t ic_rq_fast_f16(const ic_rotq_args& a, hipStream_t st);
hipError_t ic_rq_fast_bf16(const ic_rotq_args& a, hipStream_t st);
// without SmoothRot factors or perm
hipError_t ic_rq_fast_f16_plain(const ic_rotq_args& a, hipStream_t st);
hipError_t ic_rq_fast_bf16_plain(const ic_rotq_args& a, hipStream_t st);
// with both SmoothRot factors and perm
hipError_t ic_rq_fast_f16_both(const ic_rotq_args& a, hipStream_t st);
hipError_t ic_rq_fast_bf16_both(const ic_rotq_args& a, hipStream_t st);
// with the row normalisation of a.norm first (rq_norm_{f16,bf16}.hip)
hipError_t ic_rq_norm_f16(const ic_rotq_args& a, hipStream_t st);
hipError_t ic_rq_norm_bf16(const ic_rotq_args& a, hipStream_t st);
hipError_t ic_rq_norm_f16_both(const ic_rotq_args& a, hipStream_t st);
hipError_t ic_rq_norm_bf16_both(const ic_rotq_args& a, hipStream_t st);
