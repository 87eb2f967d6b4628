// Pieces shared by the DMA-pipelined MFMA GEMMs (gemm_i8.hip: W8A8 / W4A8,
// gemm_w4a16.hip: W4A16): the LDS row layout, the inline-assembly
// global->LDS DMA with its explicit waits, and the XCD-aware tile order.
#pragma once
#include "ic_common.h"

namespace {

constexpr int kNT = 512;  // threads per workgroup
constexpr int kBK = 128;  // bytes of one LDS row per stage (128 int8 or 64 16-bit K values)

typedef __attribute__((address_space(3))) char lds_char;

// LDS rows of 128 bytes hold 8 chunks of 16 bytes, the chunk index XOR-swizzled
// by row: the MFMA fragment reads (32 consecutive rows at chunk c and c+1) then
// run at the full ds_read_b128 rate on gfx950.
IC_DEV int swz(int row) { return (row >> 1) & 7; }
IC_DEV int lds_off(int row, int chunk) { return row * kBK + ((chunk ^ swz(row)) << 4); }

// Global -> LDS DMA of 16 (or 4) bytes per lane, from sbase + voff (a
// wave-uniform 64-bit base and a per-lane 32-bit byte offset) to M0 + 16*lane
// (4*lane).  Issued from inline assembly so that the compiler neither tracks
// it nor orders LDS accesses behind it; completion is waited for explicitly
// with wait_vm before the workgroup barrier that publishes the stage.  No
// memory clobber: the slot a DMA fills is read only after a wait_vm and a
// barrier (both compiler barriers), so LDS reads of other slots may be
// scheduled across the issue.  M0 holds no compiler value in these kernels
// (gfx950 LDS instructions do not use it).
IC_DEV void dma16(uint32_t voff, const void* sbase, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(voff), "s"(sbase)
               : "m0");
}
IC_DEV void dma4(uint32_t voff, const void* sbase, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, %2" ::"s"(lds), "v"(voff), "s"(sbase)
               : "m0");
}

// Block until at most N vector-memory operations of this wave are outstanding
// (they retire in issue order).
template <int N> IC_DEV void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
IC_DEV void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Logical tile id for hardware block id b.  Consecutive block ids are spread
// round-robin over the 8 XCDs; renumber so each XCD works on a contiguous run
// of logical tiles, then walk the run in bands of GM tile rows so neighbouring
// tiles share A rows and B columns in that XCD's L2.  With GM = 4 the 32
// tiles one XCD runs at a time span 4 tile rows x 8 tile columns, whose
// distinct A and B chunks per K-stage (4 x 32 + 8 x 8 KB for 256 x 128 W4A8
// tiles) are a third fewer than with 8 x 4 (8 x 32 + 4 x 8 KB): the L2
// misses, fed from the Infinity Cache at about a third of the L2's rate,
// are what bounds the GEMMs' operand delivery.  Measured against GM = 8
// (same process): C3 -1.3 %, Wan FFN-down W4A8 -4 %, W8A8 -4 %, C1 equal;
// GM = 2 is no better, GM = 16 up to 16 % slower.
IC_DEV void tile_coords(int b, int nb, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int xcd = b & 7, local = b >> 3;
  const int per = nb >> 3, rem = nb & 7;
  const int L = xcd < rem ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
  constexpr int GM = 4;
  const int in_group = GM * tiles_n;
  const int group = L / in_group;
  const int first_m = group * GM;
  const int gsize = min(tiles_m - first_m, GM);
  const int r = L - group * in_group;
  tm = first_m + r % gsize;
  tn = r / gsize;
}

}  // namespace
