// smoe_mfma.h — gfx950 building blocks shared by the grouped GEMM kernels:
// fp8 MFMA wrappers, direct global->LDS DMA issued as inline asm, the
// swizzled LDS tile layout and fragment reads.
#pragma once

#include "smoe_common.h"

namespace smoe {

constexpr int kBK = 128;   // K per step (= scale block)
constexpr int kRow = kBK;  // bytes per LDS tile row

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

// s_waitcnt with vmcnt = n (n < 16), expcnt not waited on, lgkmcnt(0): the
// encoding is vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8].
template <int n>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(n >= 0 && n < 16, "vmcnt immediate");
  __builtin_amdgcn_s_waitcnt(n | (7 << 4));
}

// Direct global->LDS loads issued as inline asm: lane i's 16 (or 4) bytes at
// base + voff land at LDS address m0 + i*16 (i*4).  The compiler does not see
// these as LDS writes, so it inserts no vmcnt(0) before the fragment reads of
// other stages; completion is tracked explicitly with s_waitcnt vmcnt(n)
// followed by a workgroup barrier.  No compiler-visible global loads are
// issued inside the K loop, so the counts are exact.
__device__ __forceinline__ void dma16(const void* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(voff),
               "s"(base)
               : "memory");
}
__device__ __forceinline__ void dma4(const void* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, %2" ::"s"(lds), "v"(voff),
               "s"(base)
               : "memory");
}

// A pointer the compiler cannot prove wave-uniform (e.g. chosen by wave
// index), moved to scalar registers for the DMA's SGPR base operand.
template <class T>
__device__ __forceinline__ const T* uniform_ptr(const T* p) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const T*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

// LDS tile layout.  ds_read_b128 serves a wave in 16-lane groups, and within
// a group lanes 0-7 and lanes 8-15 are each conflict-free only when their
// eight 16-byte accesses fall in one 128-byte half of the 64-bank array
// (address bit 7 constant) at eight distinct positions (measured with the
// LDS bank-conflict counter on gfx950).  A fragment read gives lane l tile
// row base + l%16, so tile rows r and r+8 of each 16-row group share one
// 256-byte line: row r sits at row position 2*(r&7) + (r>>3 & 1), which puts
// rows 0-7 in the low halves and rows 8-15 in the high halves; within a row
// the 16-byte chunk c is stored at slot c ^ (r & 7).
__device__ __forceinline__ int lds_row(int r) {
  return (r & ~15) | ((r & 7) << 1) | ((r >> 3) & 1);
}
// Inverse of lds_row: the tile row held at row position p.
__device__ __forceinline__ int tile_row(int p) {
  return (p & ~15) | ((p & 1) << 3) | ((p & 15) >> 1);
}
__device__ __forceinline__ int swz(int row, int chunk) {
  return lds_row(row) * kRow + ((chunk ^ (row & 7)) << 4);
}

__device__ __forceinline__ v4f mfma16(v8i a, v8i b, v4f c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

__device__ __forceinline__ v8i lds_frag(const uint8_t* base, int row, int c0) {
  const v4i lo = *(const v4i*)(base + swz(row, c0));
  const v4i hi = *(const v4i*)(base + swz(row, c0 + 1));
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Write a bf16 output tile staged in LDS (kBM rows of kBN values, row pitch
// kCPitch bytes) to c[row0 + r][n0 ..] (row length N), its first `rows`
// rows and `ncols` columns.  Thread t copies 16-byte chunk t % (kBN/8) of
// rows t / (kBN/8), then every (kThreads / (kBN/8))-th row after it, eight
// LDS reads in flight before their eight stores (a loop of read, wait,
// store leaves each store behind a full LDS round trip).
template <int kThreads, int kBM, int kBN, int kCPitch>
__device__ __forceinline__ void store_staged_tile(const uint8_t* ct, uint16_t* c, int row0,
                                                  int rows, int N, int n0, int ncols, int tid) {
  constexpr int kChunks = kBN * 2 / 16;
  constexpr int kRowStep = kThreads / kChunks;
  static_assert(kThreads % kChunks == 0 && (kBM / kRowStep) % 8 == 0, "store_staged_tile shape");
  const int ch = tid % kChunks, rt = tid / kChunks;
  const bool ch_ok = ch * 8 < ncols;
  uint8_t* dst = (uint8_t*)(c + (size_t)(row0 + rt) * N + n0) + ch * 16;
  const size_t dstep = (size_t)kRowStep * N * 2;
  const uint8_t* src = ct + rt * kCPitch + ch * 16;
#pragma unroll
  for (int i0 = 0; i0 < kBM / kRowStep; i0 += 8) {
    uint4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = *(const uint4*)(src + (i0 + u) * kRowStep * kCPitch);
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (ch_ok && rt + (i0 + u) * kRowStep < rows) *(uint4*)(dst + (size_t)(i0 + u) * dstep) = v[u];
  }
}

}  // namespace smoe
