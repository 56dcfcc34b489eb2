// The fused rmsnorm -> fp8 producer. Drop-in for rmsnorm_quant_slices and row_slices of the reference's
// src/kernels/elem_fast.hpp:23-26, 40-41.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace unholy::kernels {

using bf16 = uint16_t;

// Ref elem_fast.hpp:14-20: the mHC post-mix done by the producer of a row, in place on the streams x [T][hc][dim]
// (x null: not asked for); post [T][hc], comb [T][hc][hc] fp32; hc <= 4.
struct HcPostArgs {
  bf16* x = nullptr;
  const float* post = nullptr;
  const float* comb = nullptr;
  int hc = 0;
};

// Ref elem_fast.hpp:23-26: rmsnorm of rows x [rows, dim] (bf16 weights w [dim], eps) into y [rows, ldy], then, with
// q, act_quant_fp8 (block 128) of y into q [rows, dim] / qs [rows, dim / 128], in one launch. false (nothing
// launched) where the reference's is: in place, or slices not whole multiples of 256 values.
bool rmsnorm_quant_slices(const bf16* x, int ldx, const bf16* w, bf16* y, int ldy, uint8_t* q, uint8_t* qs, int rows,
                          int dim, float eps, hipStream_t st);
// Ref elem_fast.hpp:10-12: rmsnorm of rows x [rows, dim] (any dim) into y, out of place only, over (row, slice)
// workgroups; the same values as rmsnorm_quant_slices' y.
void rmsnorm_slices(const bf16* x, int ldx, const bf16* w, bf16* y, int ldy, int rows, int dim, float eps,
                    hipStream_t st);
// Ref elem_fast.hpp:21-22: the mHC post-mix out [T][hc][dim] of the rows x [T][dim] with the streams res [T][hc][dim]
// (post [T][hc], comb [T][hc][hc], hc <= 4); out may be res.
void hc_post_slices(const bf16* x, const bf16* res, const float* post, const float* comb, bf16* out, int T, int hc,
                    int dim, hipStream_t st);
// Ref elem_fast.hpp:40-41: slices per row so that a launch of `rows` rows has ~64 workgroups, each >= 256 values.
int row_slices(int rows, int dim);

}  // namespace unholy::kernels
