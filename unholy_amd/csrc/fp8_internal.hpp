// Launch descriptor of the dense fp8 GEMM kernels (not part of the public interface).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace unholy::kernels {

// C[M, N] (bf16, ldc) = A[M, K] (e4m3) x W[N, K]^T (e4m3), per-128 scales: e8m0 (sa8 [M, K/128], sw8
// [ceil(N/128), K/128]) or fp32 (sa32, sw32, same shapes).
struct Fp8GemmArgs {
  const uint8_t* a;
  const uint8_t* sa8;
  const float* sa32;
  const uint8_t* w;
  const uint8_t* sw8;
  const float* sw32;
  uint16_t* c;
  int ldc, M, N, K;
  int rows_cap;
  const uint16_t* xa = nullptr;  // raw bf16 activations [M, ldx] quantized in the GEMV (fp32 scales, M <= 16)
  int ldx = 0;
};

// Up to three column ranges on one input (gemv_w8a8_parts): range i has its own weights, e8m0 scales, output, ldc
// and width; t0[i] is its first 16-column tile in the grid (t0[n] = total tiles).
struct Fp8Parts {
  int n;
  const uint8_t* w[3];
  const uint8_t* sw[3];
  uint16_t* c[3];
  int ldc[3], N[3], t0[4];
};

void launch_fp8_skinny(const Fp8GemmArgs& a, hipStream_t st);
// M <= 64: one workgroup per 16-column tile, K split over its 8 waves (bandwidth-shaped).
void launch_fp8_gemv(const Fp8GemmArgs& a, hipStream_t st, const Fp8Parts* parts = nullptr);
// 16 < M <= 256 with fp32 scales: one workgroup per 32 x 32 output tile over the whole of K (N % 32, K <= 8192).
bool fp8_rows_fits(const Fp8GemmArgs& a);
void launch_fp8_rows(const Fp8GemmArgs& a, hipStream_t st);
// M > 64: the LDS-ring MFMA GEMM (N % 256, K % 128, ldc % 8; fp8_tiled_fits says whether a shape qualifies).
bool fp8_tiled_fits(const Fp8GemmArgs& a);
void launch_fp8_tiled(const Fp8GemmArgs& a, hipStream_t st);
// Picks the row-tile kernel (fp32 scales, 16 < M <= 256, where it fits), the small-M kernel (M <= 64), the tiled GEMM,
// or the row-group kernel for shapes the tiled one does not take.
void launch_fp8_gemm(const Fp8GemmArgs& a, hipStream_t st);

}  // namespace unholy::kernels
