// Building blocks of the LDS-ring GEMM kernels (gfx950): direct global -> LDS loads, vmcnt waits, the XCD-aware
// block mapping and the 32x32x16 bf16 MFMA.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.hpp"

namespace unholy::kernels::pipe {

typedef float v16f_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ v16f_t mfma32_bf16(uh::bf16x8 a, uh::bf16x8 b, v16f_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// The LDS byte address of a pointer into shared memory.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return uint32_t(size_t((const __attribute__((address_space(3))) uint8_t*)p));
}

__device__ __forceinline__ uint64_t uniform_ptr(const void* base) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  // readfirstlane returns int: go through uint32_t so the low word is zero-extended, not sign-extended.
  const uint32_t lo = uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(b))));
  const uint32_t hi = uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(b >> 32))));
  return uint64_t(lo) | uint64_t(hi) << 32;
}

// The active lanes of a wave copy 16 bytes each from base + voff (per lane) to LDS lds + 16 * lane. The loads count
// in vmcnt like any global load and complete in order. Issued as inline assembly: the compiler, seeing LDS written
// by global loads, would otherwise wait for all of them before every LDS read and drain the ring.
__device__ __forceinline__ void dma16(const void* base, uint32_t voff, uint32_t lds) {
  const uint64_t sbase = uniform_ptr(base);
  lds = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds)
               : "memory", "m0");
}
// dma16 with the nontemporal policy, for data read once (expert weights streamed from HBM by the prefill GEMM:
// 1.5-2.5% faster there). Not for data that other workgroups read again from L2 (the dense fp8 GEMM's weights, read
// by every row tile: 12% slower with it).
__device__ __forceinline__ void dma16_nt(const void* base, uint32_t voff, uint32_t lds) {
  const uint64_t sbase = uniform_ptr(base);
  lds = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(voff), "s"(sbase), "s"(lds)
               : "memory", "m0");
}
// dma16 of a row gather: lane source base + 16 * off16 (64-bit arithmetic, so a gathered row's byte offset may pass
// 4 GiB, where the 32-bit per-lane offset of dma16 would wrap). off16 passes through an empty asm statement at each
// call, so the compiler rebuilds the 64-bit address in two temporary registers per load instead of keeping one
// register pair per lane live across the K loop.
__device__ __forceinline__ void dma16_g(const void* base, uint32_t off16, uint32_t lds) {
  asm volatile("" : "+v"(off16));
  const uint8_t* addr = static_cast<const uint8_t*>(base) + (size_t(off16) << 4);
  lds = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(addr), "s"(lds) : "memory", "m0");
}
// The same with 4 bytes per lane (to LDS lds + 4 * lane): a gather of one dword per lane.
__device__ __forceinline__ void dma4(const void* base, uint32_t voff, uint32_t lds) {
  const uint64_t sbase = uniform_ptr(base);
  lds = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(sbase), "s"(lds)
               : "memory", "m0");
}

// Global loads issued as plain instructions, outside the compiler's wait accounting: the kernel counts them itself
// (vmcnt, in issue order, with the direct loads above) and marks the registers written after its wait (vlanded), so
// that no use moves above that wait. Only for registers the compiler has no reason to copy before the wait (no loop-
// carried values, no spills).
__device__ __forceinline__ uh::v4i vload16(const void* p) {
  uh::v4i v;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(p) : "memory");
  return v;
}
__device__ __forceinline__ uint32_t vload_u8(const void* p) {
  uint32_t v;
  asm volatile("global_load_ubyte %0, %1, off" : "=v"(v) : "v"(p) : "memory");
  return v;
}
__device__ __forceinline__ uint32_t vload_u32(const void* p) {
  uint32_t v;
  asm volatile("global_load_dword %0, %1, off" : "=v"(v) : "v"(p) : "memory");
  return v;
}
template <int N>
__device__ __forceinline__ void vlanded(uh::v4i (&b)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" : "+v"(b[i]));
}
__device__ __forceinline__ void vlanded(uint32_t& x) { asm volatile("" : "+v"(x)); }

template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N < 64);
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);  // vmcnt(N), no lgkm / exp wait
}

// LDS barrier that does not wait for outstanding global loads (a register prefetch stays in flight).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
}

// XOR swizzle of a 128-byte LDS row (8 pieces of 16 bytes): row r's piece p is stored at slot r * 8 + (p ^ lds_swz(r)).
// gfx950's LDS has 64 banks of 4 bytes, and a 16-byte read serves 16 lanes per pass. The 16 rows an MFMA operand
// read touches in one pass then cover the 64 banks once: rows r and r ^ 1 sit 32 banks apart (r * 128 bytes), and
// (r >> 1) & 7 spreads the row pairs over the eight 16-byte bank groups.
__device__ __forceinline__ int lds_swz(int r) { return (r >> 1) & 7; }

// Block -> (column block bx, tile by). Workgroups go round-robin over the 8 XCDs (lin % 8); XCD x runs tiles x,
// x + 8, x + 16, ... in order, each tile's column blocks back to back, so they share that XCD's L2 and the tiles that
// exist (the first *ntiles_dev of a grid sized for the maximum) are spread evenly over the XCDs. The launcher pads
// the grid's tile count to a multiple of 8.
__device__ __forceinline__ void tile_block(int nbx, int& bx, int& by) {
  const int lin = blockIdx.y * nbx + blockIdx.x, k = lin >> 3;
  by = (k / nbx) * 8 + (lin & 7);
  bx = k % nbx;
}
inline dim3 tile_grid(int nbx, int ntiles) { return dim3(unsigned(nbx), unsigned((ntiles + 7) / 8 * 8)); }

}  // namespace unholy::kernels::pipe
