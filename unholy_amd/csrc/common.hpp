// Host error handling and small device helpers shared by the kernel files.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>

#define UH_CHECK(expr)                                                                                        \
  do {                                                                                                        \
    const hipError_t uh_err_ = (expr);                                                                        \
    if (uh_err_ != hipSuccess)                                                                                \
      throw std::runtime_error(std::string(#expr) + ": " + hipGetErrorString(uh_err_) + " (" + __FILE__ +    \
                               ":" + std::to_string(__LINE__) + ")");                                         \
  } while (0)
#define UH_CHECK_LAUNCH() UH_CHECK(hipGetLastError())

namespace uh {

inline unsigned cdiv(size_t a, size_t b) { return unsigned((a + b - 1) / b); }

// Loads through a pointer read from memory (the per-expert tables) default to flat addressing; casting to the
// global address space gives global_load instructions.
template <class T>
using gptr = const __attribute__((address_space(1))) T*;
template <class T>
__device__ __forceinline__ gptr<T> as_global(const T* p) {
  return (gptr<T>)p;
}

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

// D = A (16 x 128) x B (128 x 16) + C with per-32-block e8m0 scales on both operands (measured on gfx950):
//   8-bit operand (e4m3), lane l = (row l % 16, group g = l / 16): bytes 0..15 hold inputs 16g .. 16g + 15 and
//     bytes 16..31 hold inputs 64 + 16g .. 64 + 16g + 15 of the 128-input step;
//   4-bit operand (e2m1, low 4 dwords), lane l = (column l % 16, g): nibbles 0..31 hold inputs 32g .. 32g + 31;
//   scales: lane (row or column, g) gives the e8m0 byte (low byte of the operand) of the 32-block g, whichever
//     lanes hold that block's data;
//   C: lane l holds rows 4 (l / 16) + i, i = 0..3, of column l % 16.
__device__ __forceinline__ v4f mfma_fp8_fp4(v8i a, v4i b, int sa, int sb, v4f c) {
  const v8i bb = {b[0], b[1], b[2], b[3], 0, 0, 0, 0};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, bb, c, 0, 4, 0, sa, 0, sb);
}
// The same with both operands e4m3 (the 8-bit layout above on both sides).
__device__ __forceinline__ v4f mfma_fp8_fp8(v8i a, v8i b, int sa, int sb, v4f c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, sa, 0, sb);
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// Exact in-register dequantization with the gfx950 scaled conversions: 8 e2m1 codes (one dword, low nibble first)
// or 8 e4m3 codes (two dwords, lowest byte first) times a power-of-two scale -> 8 bf16 (every such value is a
// bf16 number: e2m1 / e4m3 have <= 4 significant bits).
__device__ __forceinline__ bf16x8 fp4x8_to_bf16(uint32_t w, float sc) {
  const auto p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 0);
  const auto p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 1);
  const auto p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 2);
  const auto p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 3);
  return bf16x8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}
__device__ __forceinline__ bf16x8 fp8x8_to_bf16(uint32_t lo, uint32_t hi, float sc) {
  const auto p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, sc, false);
  const auto p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, sc, true);
  const auto p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, sc, false);
  const auto p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, sc, true);
  return bf16x8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}
// C += A (16 x 32 bf16) x B (32 x 16 bf16), fp32 accumulation. A and B lanes (row / column l % 16, group l / 16)
// hold 8 inputs each, with the same input permutation on both sides; C as above. The products are exact and the
// sums fp32: measured against fp64 this stays at fp32 accuracy (the block-scaled f8f6f4 MFMA above does not: its
// internal sums lose bits, ~3e-3 of the output at the 2^-8 rms floor).
__device__ __forceinline__ v4f mfma_bf16(bf16x8 a, bf16x8 b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

}  // namespace uh
