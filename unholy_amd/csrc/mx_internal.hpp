// Launch descriptors shared between the MXFP4 kernel files (not part of the public interface).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "unholy/kernels/exl3_moe.hpp"

namespace unholy::kernels {

// One grouped GEMV / GEMM launch: activations as e4m3 codes + e8m0 scales per 128 (aq, as) or fake-quantized
// bf16 (xa); one or two projections (index 1 null: one); optional SwiGLU epilogue (hh and/or hq + hs).
struct MxGemvArgs {
  const uint8_t* aq;
  const uint8_t* as;
  const uint16_t* xa;
  const int32_t* x_rows;  // activation mode 2: pair row r reads token row x_rows[r] of x (xa, row stride ldx)
  int ldx;
  int K, N, ldo;
  const Exl3Tile* tiles;
  int ntiles;  // tiles the grid covers (set by the launcher; the grid may be padded past it)
  const int* ntiles_dev;
  const uint8_t* const* w_tab[2];
  const uint8_t* const* s_tab[2];
  uint16_t* out[2];
  float* out32;  // non-null: projection 0 written as fp32 (before bf16 rounding) instead
  int rows_cap;
  const float* gw;
  const int32_t* grow_expert;
  const uint8_t* const* gs_tab;
  uint16_t* hh;
  uint8_t* hq;
  uint8_t* hs;
  uint16_t* hraw;  // SwiGLU rows as bf16, not requantized (MxGlu::h)
  float limit;
  // > 0: one matrix, two column streams per wave: projection 1 is projection 0's matrix from 16-column tile `split`
  // on (codes, scales and outputs offset by split tiles); the grid covers split tiles.
  int split;
};

// amode: 0 e4m3 codes + scales, 1 fake-quantized bf16 rows, 2 raw bf16 token rows (act_quant in the kernel).
void launch_mx_gemv(const MxGemvArgs& a, int ntiles, int amode, hipStream_t st);
// Exhaustive check of the hardware e4m3 encode against the software one on [-448, 448]; returns the mismatches
// (*total: values compared).
unsigned long long fp8_check_encode(unsigned long long* total);
// Exhaustive check of the hardware bf16 rounding against f32_to_bf16 over all fp32 bit patterns; returns the
// mismatches at non-NaN inputs (*nan_bad: at NaN inputs).
unsigned long long bf16_check_encode(unsigned long long* nan_bad);
// Zeroes n int32 words (a kernel, so that a captured graph records no memset node).
void launch_zero_words(int32_t* p, size_t n, hipStream_t st);
struct MoePlan;
// remote_combine over rows of stride ld (the grid strides over the device-side token count; max_tokens only sizes it).
void launch_remote_combine(const uint16_t* pair_out, int ld, const int32_t* u2p, const MoePlan* plan, uint16_t* dst,
                           int K, int dim, int max_tokens, hipStream_t st);
void launch_mx_gemm(const MxGemvArgs& a, int ntiles, int amode, hipStream_t st);
void launch_mx_transform(int mode, const uint16_t* x, int ldx, const int32_t* x_rows, const uint16_t* u,
                         const float* w, float limit, const int32_t* row_expert, const uint8_t* const* s_tab,
                         uint16_t* out, uint8_t* q, uint8_t* qs, int K, int P, hipStream_t st);

// h = bf16(SwiGLU(g, u)) (no routing weight) of M rows x I, act_quant per 128 into q / qs (and / or fake-quantized
// bf16 into hh): the second half of gemv_w8a8_glu.
void launch_swiglu_quant(const uint16_t* g, int ldg, const uint16_t* u, int ldu, int M, int I, float limit,
                         uint16_t* hh, uint8_t* q, uint8_t* qs, hipStream_t st);

}  // namespace unholy::kernels
