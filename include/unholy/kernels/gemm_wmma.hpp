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
// Ref gemm_wmma.hpp:24-26: grouped "mgk,grk->mgr" with fp8 weights x 128x128 e8m0 scales (dequantized to bf16,
// exact): a bf16 [M, G, K], w e4m3 [G R, K], sw [ceil(G R / 128), K / 128], c bf16 [M, G, R]; K % 128 == 0. M <= 384
// takes the row-tile kernel (M <= 16: R % 32 == 0, K <= 8192; else R % 64 == 0, K <= 4096), or else up to M = 160 the
// GEMV (R % 16 == 0); larger M the tiled MFMA GEMM (R % 128 == 0); other shapes the reference-order kernel.
void gemm_grouped_fp8w_wmma(const bf16* a, const uint8_t* w, const uint8_t* sw, bf16* c, int M, int G, int R, int K,
                            hipStream_t st);

}  // namespace unholy::kernels
