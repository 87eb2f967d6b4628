// W4A16: fp16/bf16 activations x INT4 weights dequantized on the fly (gfx950).
//
// Replaces unpack_int4_to_float16 (triton_int4_unpack.py:25-88) followed by the
// cuBLAS F.linear of _forward_int4_w4a16 (_ops.py:466-481): the dequantized
// weight w[n,k] = RN_dt(q[n,k] * RN_dt(s[n, k/gs])) is never written to HBM.
// Shapes with M > 128, groups of whole 64-column blocks and an aligned 16-bit
// output run gemm_i8_big_kernel's W4A16 mode (weights dequantized in registers,
// v_mfma_f32_16x16x32); the kernel below covers the rest: the dequantized tile
// is produced in LDS and consumed by v_mfma_f32_32x32x16_{f16,bf16}.  For
// fp16 this is bit-identical to the reference unpack (an fp16 product of two
// fp16 values); the reference rejects bf16 here and its PyTorch fallback
// rounds q*s to the activation type, which is what bf16 does.  Accumulation is
// fp32 in the MFMA; the epilogue adds the bias (the reference drops it on this
// path) and rounds to the activation type.
//
// The pipeline is the one of the INT8 GEMM (gemm_i8.hip, shared pieces in
// gemm_common.h): 512-thread workgroups, a 256 x 256 output tile, an NS-deep
// LDS ring filled by inline-assembly global->LDS DMAs issued in slices between
// the MFMA K-steps, explicit vmcnt waits.  One stage is 64 K values: a 128-byte
// row of 16-bit activations, 32 bytes of packed weights per output column and
// two fp32 scales per column, those of the groups of the stage's two 32-K
// halves (group sizes that are multiples of 32).  Once per stage the
// workgroup dequantizes the packed tile into a 16-bit LDS tile with the same
// swizzled row layout as the activations (two or three VALU instructions per
// weight with packed 16-bit math), then every wave runs its MFMAs from LDS.
//
// Also provides the standalone unpack kernels (INT4->int8 and INT4->fp16/bf16),
// triton_int4_to_int8_unpack.py:26-81 and triton_int4_unpack.py:25-88.
#include "dequant4.h"
#include "gemm_common.h"
#include "gemm_i8_big.h"

namespace {

IC_DEV int nib(uint32_t w, int i) {  // i-th nibble (low nibble first), two's complement
  const int v = (w >> (4 * i)) & 0xf;
  return v >= 8 ? v - 16 : v;
}

// One dequantized weight value RN_dt(q * RN_dt(s)), as f32.
template <int DT> IC_DEV float deq1(int q, float s) {
  if constexpr (DT == IC_DTYPE_F16) return (float)((_Float16)q * (_Float16)s);
  else return bf16_to_f32(f32_to_bf16((float)q * bf16_to_f32(f32_to_bf16(s))));
}
template <int DT> IC_DEV u16 deq1_bits(int q, float s) {
  if constexpr (DT == IC_DTYPE_F16) return __builtin_bit_cast(u16, (_Float16)((_Float16)q * (_Float16)s));
  else return f32_to_bf16((float)q * bf16_to_f32(f32_to_bf16(s)));
}

// W4A16 tile: BM x BN outputs, WGM wave rows, NS-deep ring of 64-K stages.
template <int BM_, int BN_, int WGM_, int NS_>
struct WTile {
  static constexpr int BM = BM_, BN = BN_, WGM = WGM_, NS = NS_;
  static constexpr int A_BYTES = BM * kBK;  // 64 16-bit activations per row
  static constexpr int B_BYTES = BN * 32;   // 64 packed INT4 weights per column
  static constexpr int S_BYTES = BN * 4;    // fp32 scale per column of one 32-K half's group
  static constexpr int SLOT = A_BYTES + B_BYTES + 2 * S_BYTES;
  static constexpr int BU_BYTES = BN * kBK;  // dequantized 16-bit weights
  static constexpr int EPI_RS = BN + 8;      // output staging row stride (elements)
  static constexpr size_t epi_bytes() { return (size_t)BM * EPI_RS * 2 + (size_t)BN * 4; }
  static constexpr size_t ring_bytes() { return (size_t)NS * SLOT + (size_t)BU_BYTES; }
  static constexpr size_t lds_bytes() { return ring_bytes() > epi_bytes() ? ring_bytes() : epi_bytes(); }
};

template <class TL, int DT>
__global__ __launch_bounds__(kNT, 1) void gemm_w4a16_kernel(
    const u16* __restrict__ A, int64_t lda, const uint8_t* __restrict__ B, int64_t ldb,
    const float* __restrict__ s_w, int G, int gsize, const void* __restrict__ bias, int bias_dt,
    u16* __restrict__ C, int64_t ldc, int M, int N, int K) {
  constexpr int BM = TL::BM, BN = TL::BN, WGM = TL::WGM, NS = TL::NS;
  constexpr int WGN = 8 / WGM;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int A_DMA = BM / 64;         // 1 KB DMA blocks of A per wave per stage
  constexpr int B_BLK = BN * 32 / 1024;  // 1 KB blocks of packed weights per stage
  constexpr int B_DMA = (B_BLK + 7) / 8; // per wave (the first B_BLK % 8 waves take one more)
  constexpr int S_WAVES = BN / 64;       // waves issuing one scale DMA per stage
  constexpr int D = A_DMA + B_DMA;
  constexpr int kParts = 4;              // DMA slices per stage (one per MFMA K-step)
  constexpr int PKC = BN * 2;            // packed 16-byte chunks dequantized per stage
  static_assert(TM >= 1 && TN >= 1 && A_DMA >= 1 && BM % 64 == 0 && BN % 32 == 0, "tile shape");
  static_assert(PKC % kNT == 0 || (B_BLK % 8 != 0 && NS == 2 && PKC % 64 == 0 && PKC < 2 * kNT),
                "dequant split: whole chunks per thread, or whole waves of chunks with a two-slot ring "
                "(the waits are then vmcnt(0))");
  static_assert(NS >= 2 && S_WAVES <= 8, "ring depth");

  extern __shared__ __attribute__((aligned(16))) char smem[];
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_char*)smem;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = wave / WGN, wc = wave % WGN;
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int tm, tn;
  tile_coords(blockIdx.x, tiles_m * tiles_n, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int KT = K / 64;
  const bool s_wave = wave < S_WAVES;

  // ---- DMA addressing.  A: lane L of a 1 KB block covers LDS row 8*blk + L/8,
  // chunk slot L%8, and loads global chunk (L%8) ^ swz(row).  Packed B: 32
  // rows of 32 bytes per block.  Scales: one dword per lane, column
  // n0 + 64*wave + lane of the stage's group.
  const int64_t lda_b = lda * 2;
  uint32_t a_off[A_DMA];
#pragma unroll
  for (int c = 0; c < A_DMA; ++c) {
    const int row = 8 * (wave + 8 * c) + (lane >> 3);
    a_off[c] = (uint32_t)(min(row, M - 1 - m0) * lda_b + (((lane & 7) ^ swz(row)) << 4));
  }
  uint32_t b_off[B_DMA];
#pragma unroll
  for (int c = 0; c < B_DMA; ++c) {
    const int row = 32 * (wave + 8 * c) + (lane >> 1);
    b_off[c] = (uint32_t)(min(row, N - 1 - n0) * ldb + ((lane & 1) << 4));
  }
  const uint32_t s_off = (uint32_t)(min(64 * wave + lane, N - 1 - n0) * G * 4);
  const char* a_base = (const char*)(A + (int64_t)m0 * lda);
  const uint8_t* b_base = B + (int64_t)n0 * ldb;
  const float* s_base = s_w + (int64_t)n0 * G;

  // kt_slot may run past the end of K: the slot stays kt_slot % NS (the one
  // the current step frees) and only the source is clamped to the last stage.
  auto issue_dma_part = [&](int kt_slot, int part) {
    const uint32_t slot = lds0 + (uint32_t)((kt_slot % NS) * TL::SLOT);
    const int kt = __builtin_amdgcn_readfirstlane(min(kt_slot, KT - 1));  // wave-uniform
    const char* ab = a_base + (int64_t)kt * kBK;
#pragma unroll
    for (int c = 0; c < A_DMA; ++c)
      if (c % kParts == part) dma16(a_off[c], ab, slot + (uint32_t)((wave + 8 * c) * 1024));
    const uint8_t* bb = b_base + (int64_t)kt * 32;
#pragma unroll
    for (int c = 0; c < B_DMA; ++c)
      if ((A_DMA + c) % kParts == part && (B_BLK % 8 == 0 || wave + 8 * c < B_BLK))  // wave-uniform
        dma16(b_off[c], bb, slot + (uint32_t)(TL::A_BYTES + (wave + 8 * c) * 1024));
    if (part == kParts - 1 && s_wave) {
      // the groups of the stage's two 32-K halves (the same one unless the
      // group size is an odd multiple of 32)
      const int g0 = G > 1 ? (kt * 64) / gsize : 0, g1 = G > 1 ? (kt * 64 + 32) / gsize : 0;
      dma4(s_off, s_base + g0, slot + (uint32_t)(TL::A_BYTES + TL::B_BYTES + wave * 256));
      dma4(s_off, s_base + g1, slot + (uint32_t)(TL::A_BYTES + TL::B_BYTES + TL::S_BYTES + wave * 256));
    }
  };
  auto issue_dma = [&](int kt) {
#pragma unroll
    for (int p = 0; p < kParts; ++p) issue_dma_part(kt, p);
  };
  // Every step issues a full stage (past the end of K a redundant reload of
  // the last stage's bytes into the slot the step frees, which nothing reads; drained
  // before the epilogue), so the stages after s always hold NS-2 steps of DMAs
  // and the DMA issue needs no branch between the MFMA K-steps.
  auto wait_stage = [&](int s) {
    if (s_wave) wait_vm<(D + 2) * (NS - 2)>();
    else wait_vm<D * (NS - 2)>();
  };

  // ---- packed INT4 -> 16-bit weights in LDS, 32 values per thread (one
  // barrier at the top of each step orders the MFMA reads of step s-1 before
  // the dequantization of step s)
  auto dequant = [&](int kt) {
    const char* slot = smem + (kt % NS) * TL::SLOT;
    char* bu = smem + NS * TL::SLOT;
#pragma unroll
    for (int h = 0; h < (PKC + kNT - 1) / kNT; ++h) {
      const int idx = tid + kNT * h;  // packed chunk: row idx/2, half idx%2
      if (PKC % kNT != 0 && idx >= PKC) break;  // wave-uniform (whole waves past the end)
      const int row = idx >> 1, part = idx & 1;
      const v4u p = *(const v4u*)(slot + TL::A_BYTES + idx * 16);
      const DeqScale d = deq_scale<DT>(((const float*)(slot + TL::A_BYTES + TL::B_BYTES + part * TL::S_BYTES))[row]);
      const uint32_t pw[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t o[4];
        deq8<DT>(pw[i], d, o);
        *(v4u*)(bu + lds_off(row, 4 * part + i)) = v4u{o[0], o[1], o[2], o[3]};
      }
    }
  };

  v16f acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = v16f{};

  auto mfma_stage = [&](int kt, int dma_kt) {
    const char* sA = smem + (kt % NS) * TL::SLOT;
    const char* sB = smem + NS * TL::SLOT;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      v4u a[TM], b[TN];
      const int ch = 2 * ks + (lane >> 5);
#pragma unroll
      for (int i = 0; i < TM; ++i) a[i] = *(const v4u*)(sA + lds_off(wr * WM + i * 32 + (lane & 31), ch));
#pragma unroll
      for (int j = 0; j < TN; ++j) b[j] = *(const v4u*)(sB + lds_off(wc * WN + j * 32 + (lane & 31), ch));
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          if constexpr (DT == IC_DTYPE_F16)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, a[i]),
                                                               __builtin_bit_cast(v8h, b[j]), acc[i][j], 0, 0, 0);
          else
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a[i]),
                                                                __builtin_bit_cast(v8bf, b[j]), acc[i][j], 0, 0, 0);
        }
      issue_dma_part(dma_kt, ks);
    }
  };

  // ---- prologue: NS-1 stages in flight; then one step per stage: make it
  // resident, dequantize its weights, run its MFMAs while refilling the slot
  // freed by the previous step
#pragma unroll
  for (int t = 0; t < NS - 1; ++t)
    issue_dma(t);
  for (int s = 0; s < KT; ++s) {
    wait_stage(s);
    lds_barrier();
    dequant(s);
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
    mfma_stage(s, s + NS - 1);
    __builtin_amdgcn_sched_barrier(0);
  }

  wait_vm<0>();  // the trailing redundant reloads land before LDS is reused
  // ---- epilogue: v = acc (+ bias), rounded once to DT
  if ((((uintptr_t)C) & 15) == 0 && (ldc & 7) == 0 && (N & 7) == 0) {
    // stage the tile through LDS row-major, then write whole rows with 16-byte stores
    constexpr int RS = TL::EPI_RS;
    lds_barrier();  // every wave is done with the last stage
    u16* ot = (u16*)smem;
    float* b_l = (float*)(smem + BM * RS * 2);
    for (int t = tid; t < BN; t += kNT) b_l[t] = bias != nullptr ? ld_any_f32(bias, bias_dt, min(n0 + t, N - 1)) : 0.0f;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int nl = wc * WN + j * 32 + (lane & 31);
      const float b = b_l[nl];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int ml = wr * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          float v = acc[i][j][r];
          if (bias != nullptr) v = v + b;
          ot[ml * RS + nl] = DT == IC_DTYPE_F16 ? f32_to_f16(v) : f32_to_bf16(v);
        }
    }
    __syncthreads();
    constexpr int CPR = BN / 8;  // 16-byte chunks per tile row
#pragma unroll 4
    for (int c = tid; c < BM * CPR; c += kNT) {
      const int row = c / CPR, col = (c % CPR) * 8;
      const int m = m0 + row, n = n0 + col;
      if (m < M && n < N) *(v4u*)(C + (int64_t)m * ldc + n) = *(const v4u*)(ot + row * RS + col);
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int n = n0 + wc * WN + j * 32 + (lane & 31);
    const float b = bias != nullptr ? ld_any_f32(bias, bias_dt, min(n, N - 1)) : 0.0f;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wr * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m >= M || n >= N) continue;
        float v = acc[i][j][r];
        if (bias != nullptr) v = v + b;
        st_from_f32<DT>(C, (int64_t)m * ldc + n, v);
      }
  }
}

// Shape-generic fallback: one thread per output, fp32 dot product.
template <int DT>
__global__ __launch_bounds__(256) void gemm_w4a16_generic_kernel(
    const u16* __restrict__ A, int64_t lda, const uint8_t* __restrict__ B, int64_t ldb,
    const float* __restrict__ s_w, int G, int gsize, const void* __restrict__ bias, int bias_dt,
    u16* __restrict__ C, int64_t ldc, int M, int N, int K) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  const int m = blockIdx.y;
  if (n >= N || m >= M) return;
  float acc = 0.0f;
  for (int k = 0; k < K; ++k) {
    const int q = nib((uint32_t)B[(int64_t)n * ldb + (k >> 1)], k & 1);
    const float w = deq1<DT>(q, s_w[(int64_t)n * G + (G > 1 ? k / gsize : 0)]);
    acc = __builtin_fmaf(ld_as_f32<DT>(A, (int64_t)m * lda + k), w, acc);
  }
  if (bias != nullptr) acc = acc + ld_any_f32(bias, bias_dt, n);
  st_from_f32<DT>(C, (int64_t)m * ldc + n, acc);
}

template <class TL, int DT>
hipError_t launch_w4a16(const u16* A, int64_t lda, const uint8_t* B, int64_t ldb, const float* s_w,
                        int G, int gsize, const void* bias, int bias_dt, u16* C, int64_t ldc, int M,
                        int N, int K, hipStream_t st) {
  const int tiles = ((M + TL::BM - 1) / TL::BM) * ((N + TL::BN - 1) / TL::BN);
  const size_t shm = TL::lds_bytes();
  static_assert(TL::lds_bytes() <= 160 * 1024, "LDS budget");
  auto kern = gemm_w4a16_kernel<TL, DT>;
  static unsigned char lds_set[64];  // per device
  if (hipError_t e = ic_set_lds_limit((const void*)kern, (int)shm, lds_set)) return e;
  kern<<<dim3(tiles), dim3(kNT), shm, st>>>(A, lda, B, ldb, s_w, G, gsize, bias, bias_dt, C, ldc, M, N, K);
  return hipGetLastError();
}

// W4A16 on the 256/288/320 x 192 tiles of gemm_i8_big_kernel (its W16 mode):
// each wave dequantizes its own weight fragments in registers beside its
// v_mfma_f32_16x16x32 instructions, so no dequantized tile is written to or
// read back from LDS and a stage has one barrier.
template <int DT, int TMB, int MODE, bool STG>
hipError_t launch_w4a16_big_t(const u16* A, int64_t lda, const uint8_t* B, int64_t ldb, const float* s_w, int G,
                              const void* bias, int bias_dt, u16* C, int64_t ldc, int M, int N, int K,
                              hipStream_t st) {
  using RT = big::Rows<TMB, MODE>;
  const int tiles = ((M + RT::BM - 1) / RT::BM) * ((N + RT::BN - 1) / RT::BN);
  auto kern = gemm_i8_big_kernel<DT, false, MODE, TMB, STG>;
  constexpr size_t shm = RT::lds_bytes;
  static unsigned char lds_set[64];  // per device
  if (hipError_t e = ic_set_lds_limit((const void*)kern, (int)shm, lds_set)) return e;
  kern<<<dim3(tiles), dim3(kNT), shm, st>>>((const int8_t*)A, lda * 2, B, ldb, nullptr, s_w, G, bias, bias_dt, C,
                                            ldc, M, N, K, ic_epi{});
  return hipGetLastError();
}

// Tile shape by workgroup rounds x tile area x relative cost per output, as
// for the INT8 big tiles: 256, 288 or 320 rows on 192 columns, or 256 or 288
// rows on 256 columns (the 320 x 256 staging tile does not fit in LDS), whose
// stages move a quarter fewer activation bytes per output: 0.95 of the
// 192-column cost per output (measured on MI355X where both take the same
// rounds x area, C2 4608 x 12288 x 3072: f16 297 -> 284 us, bf16 309 -> 296
// us, bit-identical; forced onto shapes where they take more rounds x area,
// 4608 x 3072 x 3072 75 -> 79 us, 4096 x 5120 x 5120 216 -> 258 us).
constexpr int kW16WidePct = 95;
template <int DT, int NARROW, int WIDE, bool STG>
hipError_t launch_w4a16_big_m(const u16* A, int64_t lda, const uint8_t* B, int64_t ldb, const float* s_w, int G,
                              const void* bias, int bias_dt, u16* C, int64_t ldc, int M, int N, int K, hipStream_t st) {
  const int64_t cus = ic_num_cus();
  auto cost = [&](int bm, int bn, int pct) {
    const int64_t t = (int64_t)((M + bm - 1) / bm) * ((N + bn - 1) / bn);
    return (t + cus - 1) / cus * bm * bn * pct;
  };
  const int64_t c9 = cost(288, 192, 100), c8 = cost(256, 192, 105), c10 = cost(320, 192, 99);
  const int64_t w9 = cost(288, 256, kW16WidePct), w8 = cost(256, 256, kW16WidePct * 105 / 100);
  const int64_t cn = std::min(c9, std::min(c8, c10)), cw = std::min(w9, w8);
  if (cw < cn) {
    if (w8 < w9)
      return launch_w4a16_big_t<DT, 8, WIDE, STG>(A, lda, B, ldb, s_w, G, bias, bias_dt, C, ldc, M, N, K, st);
    return launch_w4a16_big_t<DT, 9, WIDE, STG>(A, lda, B, ldb, s_w, G, bias, bias_dt, C, ldc, M, N, K, st);
  }
  if (c8 < c9 && c8 <= c10)
    return launch_w4a16_big_t<DT, 8, NARROW, STG>(A, lda, B, ldb, s_w, G, bias, bias_dt, C, ldc, M, N, K, st);
  if (c10 < c9)
    return launch_w4a16_big_t<DT, 10, NARROW, STG>(A, lda, B, ldb, s_w, G, bias, bias_dt, C, ldc, M, N, K, st);
  return launch_w4a16_big_t<DT, 9, NARROW, STG>(A, lda, B, ldb, s_w, G, bias, bias_dt, C, ldc, M, N, K, st);
}
// the three-slot ring past K = 8192 (128 stages; at 8192 the two-slot ring
// measured 188 against 192 us for 4096 x 3072, at 12288 316 against 356 us)
template <int DT, bool STG = false>
hipError_t launch_w4a16_big(const u16* A, int64_t lda, const uint8_t* B, int64_t ldb, const float* s_w, int G,
                            const void* bias, int bias_dt, u16* C, int64_t ldc, int M, int N, int K, hipStream_t st) {
  if (K > 8192)
    return launch_w4a16_big_m<DT, big::W16L, big::W16LX, STG>(A, lda, B, ldb, s_w, G, bias, bias_dt, C, ldc, M, N, K,
                                                              st);
  return launch_w4a16_big_m<DT, big::W16, big::W16X, STG>(A, lda, B, ldb, s_w, G, bias, bias_dt, C, ldc, M, N, K, st);
}

template <int DT>
hipError_t run_w4a16(const u16* A, int64_t lda, const uint8_t* B, int64_t ldb, const float* s_w, int G,
                     int gsize, const void* bias, int bias_dt, u16* C, int64_t ldc, int M, int N, int K,
                     bool mfma_ok, bool big_ok, hipStream_t st) {
  if (mfma_ok) {
    if (M > 128 && big_ok) return launch_w4a16_big<DT>(A, lda, B, ldb, s_w, G, bias, bias_dt, C, ldc, M, N, K, st);
    if (M > 128) {
      // rounds of workgroups x tile area x relative cost per output: 384 x 192 tiles (wave tiles of
      // 96 x 96, a two-slot ring) where they fill the CUs in fewer rounds, e.g. 4608 x 12288: 768
      // tiles, three rounds, against 864 of 256 x 256 (four).  Per output they cost ~5 % more than
      // 256 x 256 (more activation bytes per stage), but dequantize fewer weights per output than
      // the 192 x 384 tile of the same area, which measured 11 % slower at that shape.
      const int64_t cus = ic_num_cus();
      auto cost = [&](int bm, int bn, int pct) {
        const int64_t t = (int64_t)((M + bm - 1) / bm) * ((N + bn - 1) / bn);
        return (t + cus - 1) / cus * bm * bn * pct;
      };
      if (cost(384, 192, 105) < cost(256, 256, 100))
        return launch_w4a16<WTile<384, 192, 4, 2>, DT>(A, lda, B, ldb, s_w, G, gsize, bias, bias_dt, C, ldc, M, N, K, st);
      return launch_w4a16<WTile<256, 256, 2, 3>, DT>(A, lda, B, ldb, s_w, G, gsize, bias, bias_dt, C, ldc, M, N, K, st);
    }
    return launch_w4a16<WTile<128, 256, 2, 4>, DT>(A, lda, B, ldb, s_w, G, gsize, bias, bias_dt, C, ldc, M, N, K, st);
  }
  dim3 grid((unsigned)((N + 255) / 256), (unsigned)M);
  gemm_w4a16_generic_kernel<DT><<<grid, dim3(256), 0, st>>>(A, lda, B, ldb, s_w, G, gsize, bias, bias_dt, C, ldc, M, N, K);
  return hipGetLastError();
}

__global__ void unpack_i8_kernel(const uint8_t* __restrict__ P, int64_t ldp, int8_t* __restrict__ O,
                                 int64_t ldo, int N, int K) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)N * K;
  if (idx >= total) return;
  const int n = (int)(idx / K), k = (int)(idx % K);
  const int v = (P[(int64_t)n * ldp + (k >> 1)] >> (4 * (k & 1))) & 0xf;
  O[(int64_t)n * ldo + k] = (int8_t)(v >= 8 ? v - 16 : v);
}

template <int DT>
__global__ void unpack_fp_kernel(const uint8_t* __restrict__ P, int64_t ldp, const float* __restrict__ s_w,
                                 int G, int gsize, u16* __restrict__ O, int64_t ldo, int N, int K) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)N * K;
  if (idx >= total) return;
  const int n = (int)(idx / K), k = (int)(idx % K);
  const int q = nib((uint32_t)P[(int64_t)n * ldp + (k >> 1)], k & 1);
  O[(int64_t)n * ldo + k] = deq1_bits<DT>(q, s_w[(int64_t)n * G + (G > 1 ? k / gsize : 0)]);
}

// Staged operand layout of the big-tile W4A16 path (gemm_i8_big_kernel with
// KIL in a W4A16 mode): packed weights stage-major, O[(s * N + n) * 32 + b] =
// P[n * ldp + 32 * s + b] for 64-K stage s (16 bytes per thread), and
// scales group-major, O[g * N + n] = S[n * G + g].
__global__ void w4a16_stage_w_kernel(const uint8_t* __restrict__ P, int64_t ldp, uint8_t* __restrict__ O, int N,
                                     int S) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // 16-byte unit of O
  if (idx >= (int64_t)S * N * 2) return;
  const int64_t s = idx / (2 * (int64_t)N);
  const int r = (int)(idx - s * 2 * N);
  const uint4 v = *(const uint4*)(P + (int64_t)(r >> 1) * ldp + 32 * s + 16 * (r & 1));
  *(uint4*)(O + idx * 16) = v;
}

__global__ void w4a16_stage_s_kernel(const float* __restrict__ S, float* __restrict__ O, int N, int G) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)N * G) return;
  const int g = (int)(idx / N), n = (int)(idx % N);
  O[idx] = S[(int64_t)n * G + g];
}

}  // namespace

extern "C" {

int ic_gemm_w4a16(const void* x, int dtype, int64_t M, int64_t K, int64_t ldx, const uint8_t* w_packed,
                  int64_t N, int64_t ldw, const float* s_w, int64_t num_groups, const void* bias,
                  int bias_dtype, void* out, int64_t ldo, void* stream) {
  const char* who = "ic_gemm_w4a16";
  if (dtype != IC_DTYPE_F16 && dtype != IC_DTYPE_BF16)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: activation dtype must be f16/bf16", who);
  if (M < 0 || N <= 0 || K <= 0 || ldx < K || ldo < N || ldw * 2 < K || num_groups < 1 ||
      K % num_groups != 0)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: bad shape M=%lld N=%lld K=%lld groups=%lld", who,
                        (long long)M, (long long)N, (long long)K, (long long)num_groups);
  if (bias && bias_dtype != IC_DTYPE_F16 && bias_dtype != IC_DTYPE_BF16 && bias_dtype != IC_DTYPE_F32)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: bias dtype must be f16/bf16/f32", who);
  if (M == 0) return IC_OK;
  if (!x || !w_packed || !s_w || !out) return ic_set_error(IC_ERR_INVALID_ARG, "%s: null pointer", who);
  if (ic_gemv_applicable(M, K, x, ldx * 2, w_packed, ldw) && (num_groups == 1 || (K / num_groups) % 32 == 0))
    return ic_gemv_w4a16(x, dtype, M, K, ldx, w_packed, N, ldw, s_w, num_groups, bias, bias_dtype, out, ldo, stream);
  const int G = (int)num_groups, gsize = (int)(K / num_groups);
  // DMA pipeline: 64-K stages, scale groups of whole 32-K halves, 16-byte aligned
  // rows; 32-bit DMA offsets within one tile (activation tiles of up to 384
  // rows, weight tiles of up to 256 columns)
  const bool mfma_ok = (K % 64 == 0) && (G == 1 || gsize % 32 == 0) && !((uintptr_t)x & 15) &&
                       !((uintptr_t)w_packed & 15) && !((ldx * 2) & 15) && !(ldw & 15) &&
                       384 * ldx * 2 < (1LL << 31) && 256 * ldw < (1LL << 31) && N * G * 4 < (1LL << 31);
  // the big tiles: one scale per column and 64-K stage (groups of whole
  // stages), 320-row DMA offsets in 32 bits, and the staged output path
  // (16-byte aligned output, row stride and N multiples of 8)
  const bool big_ok = mfma_ok && (G == 1 || gsize % 64 == 0) && 320 * ldx * 2 < (1LL << 31) &&
                      320 * ldw < (1LL << 31) && !((uintptr_t)out & 15) && (ldo & 7) == 0 && (N & 7) == 0;
  hipStream_t st = (hipStream_t)stream;
  hipError_t e = dtype == IC_DTYPE_F16
                     ? run_w4a16<IC_DTYPE_F16>((const u16*)x, ldx, w_packed, ldw, s_w, G, gsize, bias, bias_dtype,
                                               (u16*)out, ldo, (int)M, (int)N, (int)K, mfma_ok, big_ok, st)
                     : run_w4a16<IC_DTYPE_BF16>((const u16*)x, ldx, w_packed, ldw, s_w, G, gsize, bias, bias_dtype,
                                                (u16*)out, ldo, (int)M, (int)N, (int)K, mfma_ok, big_ok, st);
  if (e != hipSuccess) return ic_set_error(IC_ERR_LAUNCH, "%s: %s", who, hipGetErrorString(e));
  return IC_OK;
}

int ic_w4a16_stage_layout(const uint8_t* w_packed, int64_t N, int64_t K, int64_t ldw, const float* s_w,
                          int64_t num_groups, uint8_t* w_staged, float* s_staged, void* stream) {
  const char* who = "ic_w4a16_stage_layout";
  if (N <= 0 || K <= 0 || K % 64 != 0 || ldw * 2 < K || num_groups < 1 || K % num_groups != 0 ||
      N * num_groups >= (1LL << 31) || N * K / 32 >= (1LL << 31))
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: bad shape N=%lld K=%lld ldw=%lld groups=%lld (K a multiple of 64)",
                        who, (long long)N, (long long)K, (long long)ldw, (long long)num_groups);
  if (!w_packed || !s_w || !w_staged || !s_staged) return ic_set_error(IC_ERR_INVALID_ARG, "%s: null pointer", who);
  if (((uintptr_t)w_packed & 15) || (ldw & 15) || ((uintptr_t)w_staged & 15))
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: packed rows and the staged copy must be 16-byte aligned", who);
  hipStream_t st = (hipStream_t)stream;
  const int64_t units = N * K / 32;  // 16-byte units
  w4a16_stage_w_kernel<<<dim3((unsigned)((units + 255) / 256)), dim3(256), 0, st>>>(w_packed, ldw, w_staged, (int)N,
                                                                                    (int)(K / 64));
  const int64_t ns = N * num_groups;
  w4a16_stage_s_kernel<<<dim3((unsigned)((ns + 255) / 256)), dim3(256), 0, st>>>(s_w, s_staged, (int)N,
                                                                                 (int)num_groups);
  return ic_check_launch(who);
}

int ic_gemm_w4a16_staged(const void* x, int dtype, int64_t M, int64_t K, int64_t ldx, const uint8_t* w_staged,
                         int64_t N, const float* s_staged, int64_t num_groups, const void* bias, int bias_dtype,
                         void* out, int64_t ldo, void* stream) {
  const char* who = "ic_gemm_w4a16_staged";
  if (dtype != IC_DTYPE_F16 && dtype != IC_DTYPE_BF16)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: activation dtype must be f16/bf16", who);
  if (M < 0 || N <= 0 || K <= 0 || ldx < K || ldo < N || num_groups < 1 || K % num_groups != 0)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: bad shape M=%lld N=%lld K=%lld groups=%lld", who, (long long)M,
                        (long long)N, (long long)K, (long long)num_groups);
  if (bias && bias_dtype != IC_DTYPE_F16 && bias_dtype != IC_DTYPE_BF16 && bias_dtype != IC_DTYPE_F32)
    return ic_set_error(IC_ERR_INVALID_ARG, "%s: bias dtype must be f16/bf16/f32", who);
  if (M == 0) return IC_OK;
  if (!x || !w_staged || !s_staged || !out) return ic_set_error(IC_ERR_INVALID_ARG, "%s: null pointer", who);
  const int G = (int)num_groups, gsize = (int)(K / num_groups);
  // the big tiles' conditions (as in ic_gemm_w4a16), and M above the GEMV
  // and small-tile range: the staged layout has no other kernel
  const bool ok = M > 128 && K % 64 == 0 && (G == 1 || gsize % 64 == 0) && !((uintptr_t)x & 15) &&
                  !((uintptr_t)w_staged & 15) && !((ldx * 2) & 15) && 320 * ldx * 2 < (1LL << 31) &&
                  N * G < (1LL << 31) && !((uintptr_t)out & 15) && (ldo & 7) == 0 && (N & 7) == 0;
  if (!ok)
    return ic_set_error(IC_ERR_INVALID_ARG,
                        "%s: the staged layout needs M > 128, K and the group size multiples of 64, N and the output "
                        "row stride multiples of 8 and 16-byte aligned operands (M=%lld N=%lld K=%lld groups=%lld); "
                        "other shapes take ic_gemm_w4a16",
                        who, (long long)M, (long long)N, (long long)K, (long long)num_groups);
  hipStream_t st = (hipStream_t)stream;
  hipError_t e = dtype == IC_DTYPE_F16
                     ? launch_w4a16_big<IC_DTYPE_F16, true>((const u16*)x, ldx, w_staged, N * 32, s_staged, G, bias,
                                                            bias_dtype, (u16*)out, ldo, (int)M, (int)N, (int)K, st)
                     : launch_w4a16_big<IC_DTYPE_BF16, true>((const u16*)x, ldx, w_staged, N * 32, s_staged, G, bias,
                                                             bias_dtype, (u16*)out, ldo, (int)M, (int)N, (int)K, st);
  if (e != hipSuccess) return ic_set_error(IC_ERR_LAUNCH, "%s: %s", who, hipGetErrorString(e));
  return IC_OK;
}

int ic_unpack_int4_to_int8(const uint8_t* packed, int64_t N, int64_t K, int64_t ldp, int8_t* out,
                           int64_t ldo, void* stream) {
  if (N < 0 || K < 0 || ldp * 2 < K || ldo < K || (N * K > 0 && (!packed || !out)))
    return ic_set_error(IC_ERR_INVALID_ARG, "ic_unpack_int4_to_int8: bad arguments");
  const int64_t total = N * K;
  if (total == 0) return IC_OK;
  unpack_i8_kernel<<<dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream>>>(
      packed, ldp, out, ldo, (int)N, (int)K);
  return ic_check_launch("ic_unpack_int4_to_int8");
}

int ic_unpack_int4_to_float(const uint8_t* packed, const float* s_w, int64_t num_groups, int64_t N,
                            int64_t K, int64_t ldp, void* out, int out_dtype, int64_t ldo, void* stream) {
  if (N < 0 || K < 0 || ldp * 2 < K || ldo < K || num_groups < 1 || (K > 0 && K % num_groups != 0) ||
      (N * K > 0 && (!packed || !out || !s_w)))
    return ic_set_error(IC_ERR_INVALID_ARG, "ic_unpack_int4_to_float: bad arguments");
  if (out_dtype != IC_DTYPE_F16 && out_dtype != IC_DTYPE_BF16)
    return ic_set_error(IC_ERR_INVALID_ARG, "ic_unpack_int4_to_float: out dtype must be f16/bf16");
  const int64_t total = N * K;
  if (total == 0) return IC_OK;
  const int G = (int)num_groups, gsize = (int)(K / num_groups);
  dim3 grid((unsigned)((total + 255) / 256));
  if (out_dtype == IC_DTYPE_F16)
    unpack_fp_kernel<IC_DTYPE_F16><<<grid, dim3(256), 0, (hipStream_t)stream>>>(packed, ldp, s_w, G, gsize, (u16*)out, ldo, (int)N, (int)K);
  else
    unpack_fp_kernel<IC_DTYPE_BF16><<<grid, dim3(256), 0, (hipStream_t)stream>>>(packed, ldp, s_w, G, gsize, (u16*)out, ldo, (int)N, (int)K);
  return ic_check_launch("ic_unpack_int4_to_float");
}

}  // extern "C"
