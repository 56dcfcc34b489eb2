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

// Ref gemv.hpp:31-35: act_quant_fp8 (block 128) outputs q [M][N] / qs [M][N / 128]. counters [N / 128] belong to the
// reference's in-launch quantization; here they are accepted, never touched, and stay zero.
struct GemvQuant {
  uint8_t* q = nullptr;
  uint8_t* qs = nullptr;
  uint32_t* counters = nullptr;
};
// Ref gemv.hpp:36-37: the grouped fp8-weight GEMV ("mgk,grk->mgr", as gemm_grouped_fp8w_wmma), M <= 32,
// K % 128 == 0; gq.q set: act_quant_fp8 (block 128) of the outputs c [M, G R] into gq.q / gq.qs ((G R) % 128 == 0;
// a second launch here, gq.counters never touched).
void gemv_grouped_fp8w(const bf16* a, const uint8_t* w, const uint8_t* sw, bf16* c, int M, int G, int R, int K,
                       hipStream_t st, const GemvQuant& gq = {});
// Ref gemv.hpp:40-49: a column range on the shared input: weights (e4m3 [N, K]), e8m0 scales [ceil(N/128), K/128],
// bf16 output [M, ldc], width N.
struct GemvPart {
  const void* w;
  const uint8_t* sw;
  void* c;
  int ldc, N;
};
struct GemvParts {
  static constexpr int kMax = 3;
  int n = 0;
  GemvPart p[kMax];
};
// Ref gemv.hpp:50-51: up to three W8A8 GEMVs on one input in one launch; every column exactly as gemv_w8a8's.
void gemv_w8a8_parts(const uint8_t* a, const uint8_t* sa, const GemvPart* parts, int nparts, int M, int K,
                     hipStream_t st);
// Ref gemv.hpp:52-56: parts[0] = gate, parts[1] = up (one width I, I % 128 == 0) into their outputs, then
// h = bf16(SwiGLU(gate, up)) with the clamp `limit` (no routing weight; kernels::swiglu's arithmetic) and
// act_quant_fp8 of h per 128 into gq.q / gq.qs. (A second launch here instead of the reference's last-block
// counters.)
void gemv_w8a8_glu(const uint8_t* a, const uint8_t* sa, const GemvPart* parts, int M, int K, float limit,
                   const GemvQuant& gq, hipStream_t st);

}  // namespace unholy::kernels
