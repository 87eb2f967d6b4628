// Peak-rate probes for bench.py on gfx950: the dense MFMA rates this GPU
// sustains at its loaded clock, measured with register-only loops (no memory
// traffic inside the timed loop).  Reported beside the published peaks, so a
// kernel's roofline fraction can be read against both.
//
//   bp_mfma_i8(iters, out, stream):  v_mfma_i32_32x32x32_i8, 65536 ops each
//   bp_mfma_f16(iters, out, stream): v_mfma_f32_32x32x16_f16, 32768 flops each
//
// Each wave runs kChains independent accumulator chains (so the MFMA pipeline
// is never waiting on a result), iters times; one value per lane is stored
// at the end so the loop cannot be removed.  The grid is bp_grid() = two
// 256-thread workgroups per CU (two waves per SIMD); `out` must hold
// bp_grid() * 256 ints.  The launchers return the hipError_t of the launch.
//
// bp_mfma_i8 also samples the shader clock: when `clk` is not null, the first
// lane of workgroup 0 stores the shader-clock counter (clock64) and the
// constant-rate wall clock (wall_clock64, bp_wall_clock_khz() ticks per ms)
// before and after its loop into clk[0..3], so the host can compute the
// engine clock the MFMA loop actually ran at.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int kThreads = 256;  // 4 waves: one per SIMD
constexpr int kChains = 4;

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

__global__ __launch_bounds__(kThreads) void mfma_i8_loop(int iters, int* __restrict__ out,
                                                         long long* __restrict__ clk) {
  const int lane = threadIdx.x & 63;
  const bool sample = clk != nullptr && blockIdx.x == 0 && threadIdx.x == 0;
  long long c0 = 0, w0 = 0;
  if (sample) {
    c0 = clock64();
    w0 = wall_clock64();
  }
  v4i a = {lane, lane + 1, lane + 2, lane + 3};
  v4i b = {lane ^ 5, lane ^ 7, lane ^ 9, lane ^ 11};
  v16i acc[kChains];
#pragma unroll
  for (int c = 0; c < kChains; ++c) acc[c] = v16i{};
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int c = 0; c < kChains; ++c) acc[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, acc[c], 0, 0, 0);
  }
  int s = 0;
#pragma unroll
  for (int c = 0; c < kChains; ++c) s += acc[c][0];
  if (sample) {  // after a use of every chain, so the loop is inside the window
    const long long c1 = clock64(), w1 = wall_clock64();
    clk[0] = c0;
    clk[1] = c1;
    clk[2] = w0;
    clk[3] = w1;
  }
  s = 0;
#pragma unroll
  for (int c = 0; c < kChains; ++c)
#pragma unroll
    for (int r = 0; r < 16; ++r) s += acc[c][r];
  out[blockIdx.x * kThreads + threadIdx.x] = s;
}

__global__ __launch_bounds__(kThreads) void mfma_f16_loop(int iters, int* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  v8h a, b;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    a[k] = (_Float16)((lane + k) & 7);
    b[k] = (_Float16)((lane ^ k) & 3);
  }
  v16f acc[kChains];
#pragma unroll
  for (int c = 0; c < kChains; ++c) acc[c] = v16f{};
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int c = 0; c < kChains; ++c) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[c], 0, 0, 0);
  }
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < kChains; ++c)
#pragma unroll
    for (int r = 0; r < 16; ++r) s += acc[c][r];
  out[blockIdx.x * kThreads + threadIdx.x] = (int)s;
}

}  // namespace

extern "C" {

// Workgroups (of 256 threads) to launch: 2 per CU, i.e. two waves per SIMD.
int bp_grid(void) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return 0;
  return 2 * cus;
}

// Ops (kind 0: i8, 65536 per MFMA) or flops (kind 1: f16, 32768 per MFMA)
// performed by one launch of `iters` iterations.
double bp_ops_per_launch(int kind, int iters) {
  return (double)bp_grid() * (kThreads / 64) * iters * kChains * (kind == 0 ? 65536.0 : 32768.0);
}

// Ticks per millisecond of the wall clock that wall_clock64() reads.
int bp_wall_clock_khz(void) {
  int dev = 0, khz = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess)
    return 0;
  return khz;
}

int bp_mfma_i8(int iters, int* out, long long* clk, void* stream) {
  const int grid = bp_grid();
  if (grid <= 0 || iters <= 0 || out == nullptr) return (int)hipErrorInvalidValue;
  mfma_i8_loop<<<dim3(grid), dim3(kThreads), 0, (hipStream_t)stream>>>(iters, out, clk);
  return (int)hipGetLastError();
}

int bp_mfma_f16(int iters, int* out, void* stream) {
  const int grid = bp_grid();
  if (grid <= 0 || iters <= 0 || out == nullptr) return (int)hipErrorInvalidValue;
  mfma_f16_loop<<<dim3(grid), dim3(kThreads), 0, (hipStream_t)stream>>>(iters, out);
  return (int)hipGetLastError();
}

}  // extern "C"
