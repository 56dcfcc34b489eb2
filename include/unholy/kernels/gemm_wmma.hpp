// Tiled fp8 W8A8 GEMM. Drop-in for gemm_w8a8_wmma of the reference's src/kernels/gemm_wmma.hpp:12-18 (there a
// gfx12 WMMA kernel; here exact e4m3 -> bf16 dequantization and the gfx950 bf16 MFMA). a e4m3 [M, K], sa e8m0 [M, K/128]; w e4m3 [N, K], sw
// e8m0 [ceil(N/128), K/128]; K % 128 == 0.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace unholy::kernels {

using bf16 = uint16_t;

void gemm_w8a8_wmma(const uint8_t* a, const uint8_t* sa, const uint8_t* w, const uint8_t* sw, bf16* c, int ldc,
                    int M, int N, int K, hipStream_t st);
void gemm_force_skinny(int on);  // the reference's test override; kernel choice here is by shape only (no-op)

}  // namespace unholy::kernels
