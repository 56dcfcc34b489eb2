// Skinny fp8 W8A8 GEMV for decode rows. Drop-in for the W8A8 entry of the reference's src/kernels/gemv.hpp
// (gemv.hpp:19-25): same contract as gemm_w8a8 (e4m3 A [M, K] + e8m0 sa [M, K/128], e4m3 W [N, K] + e8m0
// sw [ceil(N/128), K/128], bf16 C), M <= kGemvRowsCap. A row's result does not depend on M.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace unholy::kernels {

using bf16 = uint16_t;

constexpr int kGemvRowsCap = 32;
int gemv_max_rows();  // rows up to which dense layers take the GEMV (8, as the reference's default)
void gemv_w8a8(const uint8_t* a, const uint8_t* sa, const uint8_t* w, const uint8_t* sw, bf16* c, int ldc, int M,
               int N, int K, hipStream_t st);

}  // namespace unholy::kernels
