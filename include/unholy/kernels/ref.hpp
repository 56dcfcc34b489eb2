// Quantization, routing, SwiGLU and combine entry points of the reference's src/kernels/ref.hpp that lie on the
// quantized expert path, with the reference's arithmetic (ref_elem.hip, ref_moe.hip, ref_gemm.hip), plus the
// softmax top-k router and fp32-scale fp8 forms of the synthetic workload. bf16 = uint16_t, fp8 = uint8_t
// e4m3fn, scales = uint8_t e8m0 unless named *_f32s. Matrices row-major; linear weights [out, in]; C = A W^T.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace unholy::kernels {

using bf16 = uint16_t;

// act_quant(x, block): q e4m3 [rows, cols], s e8m0 [rows, cols/block]; block in {32, 64, 128}. Ref ref.hpp:128.
void act_quant_fp8(const bf16* x, int ldx, uint8_t* q, uint8_t* s, int rows, int cols, int block, hipStream_t st);
// In-place quantize + dequantize to bf16. Ref ref.hpp:130.
void fake_quant_fp8(bf16* x, int ldx, int rows, int cols, int block, hipStream_t st);
// In-place e2m1 quantize + dequantize per block (the attention indexer's query operand; block 32 there). Ref
// ref.hpp:25. block % 8 == 0 (the reference's block is 32 or a multiple), cols % block == 0.
void fake_quant_fp4(bf16* x, int ldx, int rows, int cols, int block, hipStream_t st);
// act_quant with fp32 scales (kernel.py act_quant, scale_fmt=None): s = max(amax, 1e-4) * fp32(1/448).
void act_quant_fp8_f32s(const bf16* x, int ldx, uint8_t* q, float* s, int rows, int cols, int block, hipStream_t st);

// fp8 x fp8 with e8m0 scales per 128 (sa [M, K/128], sw [ceil(N/128), K/128]). Ref ref.hpp:135-136.
void gemm_w8a8(const uint8_t* a, const uint8_t* sa, const uint8_t* w, const uint8_t* sw, bf16* c, int ldc, int M,
               int N, int K, hipStream_t st);
// fp8 x fp8 with fp32 scales: sa [M, K/128] per 1x128 activation block, sw [ceil(N/128), K/128] per 128x128
// weight block; C = sum_kb (raw_kb) * (sa * sw), fp32, bf16 out.
void gemm_fp8_f32s(const uint8_t* a, const float* sa, const uint8_t* w, const float* sw, bf16* c, int ldc, int M,
                   int N, int K, hipStream_t st);
// No reference counterpart: act_quant_fp8_f32s (block 128) of bf16 x [M, ldx] fused into gemm_fp8_f32s, M <= 16;
// the same results bit for bit in one launch (for decode rows). ldx % 8 == 0, x 16-byte aligned.
void gemm_fp8_f32s_x(const bf16* x, int ldx, const uint8_t* w, const float* sw, bf16* c, int ldc, int M, int N,
                     int K, hipStream_t st);
// Grouped "mgk,grk->mgr" with fp8 weights dequantized by 128x128 e8m0 block scales, in the reference's order (one
// fp32 fmaf chain over k per output). Ref ref.hpp:42-45. K % 128 == 0.
void gemm_grouped_fp8w(const bf16* a, const uint8_t* w, const uint8_t* sw, bf16* c, int M, int G, int R, int K,
                       hipStream_t st);
// fp8 activations x e2m1 weights [N, K/2] (row-major or the tile-major layout). Ref ref.hpp:139-143.
void gemm_a8w4(const uint8_t* a, const uint8_t* sa, const uint8_t* w, const uint8_t* sw, bf16* c, int ldc, int M,
               int N, int K, hipStream_t st);
void gemm_a8w4_tiled(const uint8_t* a, const uint8_t* sa, const uint8_t* w, const uint8_t* sw, bf16* c, int ldc,
                     int M, int N, int K, hipStream_t st);

// DSV4 router: sqrt(softplus(logit)) + bias selects K of E (hash layers: tid2eid[ids]); weights normalised times
// route_scale. Ref ref.hpp:243-249.
void route(const float* logits, const float* bias, const int32_t* tid2eid, const int32_t* ids, int32_t* sel,
           float* weights, int T, int E, int K, float route_scale, hipStream_t st, const float* bias_vl = nullptr,
           int vocab = 0);
void route_fast(const float* logits, const float* bias, const int32_t* tid2eid, const int32_t* ids, int32_t* sel,
                float* weights, int T, int E, int K, float route_scale, hipStream_t st, const float* bias_vl = nullptr,
                int vocab = 0);
// GLM router: sigmoid(logit) + bias selects, picks in ascending id, weights s / (sum s + 1e-20) * route_scale
// (the reference's glm route in moe_dispatch.hip:308-356).
void route_glm(const float* logits, const float* bias, int32_t* sel, float* weights, int T, int E, int K,
               float route_scale, hipStream_t st);
// Softmax top-K renormalised over the picks: picks by logit descending (ties to the lower id), weight
// exp(l - l_first) / sum over the picks in selection order. E <= 1024, K <= 8.
void route_softmax(const float* logits, int32_t* sel, float* weights, int T, int E, int K, hipStream_t st);

// h = bf16(w[row] * silu(min(g, lim)) * clamp(u, +-lim)); w may be null. Ref ref.hpp:251-252.
void swiglu(const bf16* gate, const bf16* up, const float* w, bf16* h, int rows, int dim, float limit,
            hipStream_t st);
void scatter_add(const bf16* src, const int32_t* rows_idx, float* y, int n, int dim, hipStream_t st);
void gather_rows(const bf16* src, const int32_t* rows_idx, bf16* dst, int n, int dim, hipStream_t st);
// out[t] = bf16(sum_j pair_out[pidx[t][j]] (j ascending) + shared[t]) in fp32; shared may be null (zero).
// Ref ref.hpp:258-259.
void moe_combine(const bf16* pair_out, const int32_t* pidx, const bf16* shared, bf16* out, int T, int K, int dim,
                 hipStream_t st);

}  // namespace unholy::kernels
