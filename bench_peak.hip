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
//
//   bp_lds_delivery(buf, bytes, iters, sink, stream): the rate at which
//   global_load_lds_dwordx4 moves data from the memory hierarchy into LDS,
//   the path the GEMMs stage their operands through.  One 512-thread
//   workgroup per CU; per iteration each wave issues 7 DMAs of 1 KB (a 56 KB
//   stage per CU, two stages in flight, as in the tiled GEMMs), from 1 KB
//   blocks of `buf` spread over the buffer.  A buffer that fits the L2
//   (2 MB) gives the L2-hit rate, one that does not (64 MB) the Infinity
//   Cache rate.  Bytes moved per launch: bp_lds_delivery_bytes(iters).
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

constexpr int kDmaPer = 7;                      // 1 KB DMAs per wave and stage
constexpr int kDmaStage = 8 * kDmaPer * 1024;   // bytes per workgroup and stage

__global__ __launch_bounds__(512, 1) void lds_delivery(const char* __restrict__ buf, long long nblk, int iters,
                                                       int* __restrict__ sink) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const unsigned lds0 = (unsigned)(uintptr_t)(__attribute__((address_space(3))) char*)smem;
  auto issue = [&](int it) {
#pragma unroll
    for (int c = 0; c < kDmaPer; ++c) {
      const long long blk = ((long long)blockIdx.x * 977 + (long long)it * 56 + wave * kDmaPer + c) % nblk;
      const char* src = buf + blk * 1024;
      const unsigned dst = lds0 + (unsigned)((it & 1) * kDmaStage + (wave * kDmaPer + c) * 1024);
      asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(dst), "v"((unsigned)(lane * 16)),
                   "s"(src) : "m0");
    }
  };
  issue(0);
  for (int it = 0; it < iters; ++it) {
    if (it + 1 < iters) {
      issue(it + 1);
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kDmaPer) : "memory");  // stage it has landed
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) sink[blockIdx.x] = smem[lane];
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

// Bytes one bp_lds_delivery launch of `iters` iterations moves into LDS.
double bp_lds_delivery_bytes(int iters) { return (double)(bp_grid() / 2) * iters * kDmaStage; }

// sink must hold bp_grid() / 2 ints; bytes >= 1 KB.
int bp_lds_delivery(const void* buf, long long bytes, int iters, int* sink, void* stream) {
  const int grid = bp_grid() / 2;
  if (grid <= 0 || iters <= 0 || buf == nullptr || sink == nullptr || bytes < 1024) return (int)hipErrorInvalidValue;
  const int shm = 2 * kDmaStage;
  hipError_t e = hipFuncSetAttribute((const void*)lds_delivery, hipFuncAttributeMaxDynamicSharedMemorySize, shm);
  if (e != hipSuccess) return (int)e;
  lds_delivery<<<dim3(grid), dim3(512), shm, (hipStream_t)stream>>>((const char*)buf, bytes / 1024, iters, sink);
  return (int)hipGetLastError();
}

int bp_mfma_f16(int iters, int* out, void* stream) {
  const int grid = bp_grid();
  if (grid <= 0 || iters <= 0 || out == nullptr) return (int)hipErrorInvalidValue;
  mfma_f16_loop<<<dim3(grid), dim3(kThreads), 0, (hipStream_t)stream>>>(iters, out);
  return (int)hipGetLastError();
}

}  // extern "C"
