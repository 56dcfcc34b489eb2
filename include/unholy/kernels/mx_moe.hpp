// MXFP4 routed-expert kernels for gfx950. Drop-in for the reference's src/kernels/mx_moe.hpp (same names,
// signatures, weight/scale layouts and pointer-table semantics; cited per entry point below).
//
// Weights: e2m1 codes (two per byte, low nibble = even input) with one e8m0 scale per 32 inputs, repacked at
// load into the tile-major layout: for 64-input slab kt and 16-output tile nt, chunk kt * (N/16) + nt holds
// 512 code bytes (output n's 32 bytes at (n % 16) * 32) and 32 scale bytes (n's two 32-blocks at (n % 16) * 2)
// (mx_moe.hpp:11-14 of the reference). Tables are [w1, w3, w2] x [codes, scales] x E device pointers; a null
// entry means the expert is not on this device and its rows are skipped (mx_moe.hpp:8-9).
//
// Arithmetic: each expert product is sum over 32-blocks of (sum of e4m3(x) * e2m1(w)) * sa * sw with sa the
// activation row's e8m0 scale per 128 inputs and sw the weight's per 32 (the reference's act_quant_fp8 +
// gemm_a8w4, ref_gemm.hip:180-183). Here both operands are dequantized exactly in registers (every e4m3 x 2^k
// and e2m1 x 2^k value is a bf16 number) and multiplied on the bf16 MFMA with fp32 accumulation: the same exact
// products summed in another fp32 order. The block-scaled f8f6f4 MFMA is only a selectable speed mode of the prefill
// GEMM (mx_gemm_set_exact(0)): its internal sums lose bits, measured at ~3e-3 of the output against fp64 on this
// hardware, outside the parity tolerance.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "unholy/kernels/exl3_moe.hpp"
#include "unholy/kernels/moe_dispatch.hpp"

namespace unholy::kernels {

using bf16 = uint16_t;

// [N, K/2] codes + [N, K/32] scales -> tile-major, in place (tmp: N*K/2 + N*K/32 bytes). Ref mx_moe.hpp:27.
void mx_repack(uint8_t* w, uint8_t* s, int N, int K, uint8_t* tmp, hipStream_t st);
// The same permutation into separate buffers. Ref mx_moe.hpp:29.
void mx_repack_to(const uint8_t* w, const uint8_t* s, uint8_t* tw, uint8_t* ts, int N, int K, hipStream_t st);

// xa[r] = bf16(fq8_128(x[x_rows ? x_rows[r] : r])) for rows whose expert is resident. Ref mx_moe.hpp:33-34.
void mx_xform_in(const bf16* x, int ldx, const int32_t* row_expert, const uint8_t* const* s_tab, bf16* xa, int P,
                 int K, hipStream_t st, const int32_t* x_rows = nullptr);
// Ref mx_moe.hpp:36-40: the same xa rows rebuilt from compact fp8 inputs (quant_remote_tokens): row r in
// [plan->remote0, plan->P) whose expert is resident (s_tab entry non-null; s_tab null: all) takes token p2u[r]'s codes
// q [U, K] and exponents s [U, K / 128]. Bit-identical to mx_xform_in on the rows those tokens would have been
// gathered into.
void mx_xform_in_q(const uint8_t* q, const uint8_t* s, const int32_t* p2u, const MoePlan* plan,
                   const int32_t* row_expert, const uint8_t* const* s_tab, bf16* xa, int P, int K, hipStream_t st);
// hh[r] = bf16(fq8_128(bf16(w[r] * silu(min(g, lim)) * clamp(u, +-lim)))). Ref mx_moe.hpp:41-42.
void mx_swiglu(const bf16* g, const bf16* u, const float* w, const int32_t* row_expert, const uint8_t* const* s_tab,
               bf16* hh, int P, int I, float limit, hipStream_t st);

// out[r] = xa[r] @ W[e]^T over each tile's rows; second projection (w3) of the same rows with w_tab2/s_tab2/out2.
// Ref mx_moe.hpp:49-52. Preconditions: K % 64 == 0 and N % 128 == 0, the reference's (mx_moe.hip:1045). max_rows:
// the caller's bound on any tile's rows; <= 64 with K % 128 == 0 runs the tiles on the grouped GEMV 16 rows at a time
// (the reference's skinny route, mx_moe.hip:1054), with the same outputs.
void mx_grouped_gemm(const bf16* xa, int K, const Exl3Tile* tiles, int ntiles, const uint8_t* const* w_tab,
                     const uint8_t* const* s_tab, bf16* out, int ldo, int N, hipStream_t st,
                     const int* ntiles_dev = nullptr, const uint8_t* const* w_tab2 = nullptr,
                     const uint8_t* const* s_tab2 = nullptr, bf16* out2 = nullptr, int max_rows = kExl3TileRows);
bool mx_skinny_enabled();
// Register-B tiles are a gfx11 design of the reference (mx_moe.hpp:54-58): false here; the setters are no-ops.
bool mx_gemm_rb();
void mx_gemm_force_rb(int on);
void mx_gemm_rb_double_buffer(int on);
// Exhaustive check of the MFMA's block-scaled decode against the closed forms: every e2m1 code x every e8m0
// scale on the weight operand, every e4m3 code x every scale on the activation operand. Returns the
// mismatches among results that are normal fp32 numbers (*total: how many were compared). Ref mx_moe.hpp:61
// (there: the v_perm dequant against the LDS table).
unsigned long long mx_check_dequant(unsigned long long* total);

constexpr int kMxGemvTileRows = 8;  // ref mx_moe.hpp:67
int mx_gemv_max_tokens();           // UNHOLY_MX_GEMV_TOKENS, default 8 (ref mx_moe.hpp:70)
inline bool mx_use_gemv(int tokens) { return tokens <= mx_gemv_max_tokens(); }

// SwiGLU (+ fake quant) in the w1/w3 launch: hh [P, N] written for every row of every tile. Ref mx_moe.hpp:74-81.
// counters is accepted for signature compatibility and not used (one workgroup holds both projections of its
// 128 outputs). hq / hs (extension): also (or instead) write hh as e4m3 codes [P, N] + e8m0 scales [P, N/128].
struct MxGlu {
  const float* w = nullptr;
  const int32_t* row_expert = nullptr;
  const uint8_t* const* s_tab = nullptr;
  bf16* hh = nullptr;
  float limit = 0.0f;
  uint32_t* counters = nullptr;
  uint8_t* hq = nullptr;
  uint8_t* hs = nullptr;
  // Extension (no reference counterpart): SwiGLU rows h = bf16(w * silu(g) * u) [P, N] without the per-128 fp8
  // requantization, for a consumer that quantizes them itself (mx_grouped_gemv_x on h gives the codes of hh exactly).
  // Excludes hh / hq; the GEMV then needs no whole-block workgroups.
  bf16* h = nullptr;
};
bool mx_gemm_glu();
void mx_gemm_force_glu(int on);
// Remote token sums (ref mx_moe.hpp:90-96): with dst, mx_grouped_gemv also writes dst[u] = bf16(sum over token u's
// remote pair rows u2p[u][j] >= 0 of out, fp32 adds in pick order) for u < plan->n_remote_tokens (N % 128; no second
// projection or GLU epilogue). Done as a second launch (remote_combine over out); counters are not used.
struct MxSums {
  const int32_t* u2p = nullptr;
  const MoePlan* plan = nullptr;
  int K = 0;
  bf16* dst = nullptr;
  uint32_t* counters = nullptr;
};
// w1 and w3 with the SwiGLU epilogue in one launch. Ref mx_moe.hpp:97-99.
void mx_grouped_gemm_glu(const bf16* xa, int K, const Exl3Tile* tiles, int ntiles, const uint8_t* const* w1_tab,
                         const uint8_t* const* s1_tab, const uint8_t* const* w3_tab, const uint8_t* const* s3_tab, int N,
                         const MxGlu& glu, hipStream_t st, const int* ntiles_dev = nullptr);
// Ref mx_moe.hpp:100-104.
void mx_grouped_gemv(const bf16* xa, int K, const Exl3Tile* tiles, int ntiles, const uint8_t* const* w_tab,
                     const uint8_t* const* s_tab, bf16* out, int ldo, int N, hipStream_t st,
                     const int* ntiles_dev = nullptr, const uint8_t* const* w_tab2 = nullptr,
                     const uint8_t* const* s_tab2 = nullptr, bf16* out2 = nullptr, int max_rows = kMxGemvTileRows,
                     const MxGlu& glu = {}, const MxSums& sums = {});

// ---- native fp8-activation forms (no reference counterpart: the activations stay as e4m3 codes + e8m0 scales
// per 128, one byte per input, instead of fake-quantized bf16) -----------------------------
// q [P, K] e4m3 + qs [P, K/128] e8m0: act_quant_fp8 of x[x_rows[r]] per 128 (rows of non-resident experts skipped).
void mx_xform_in_fp8(const bf16* x, int ldx, const int32_t* row_expert, const uint8_t* const* s_tab, uint8_t* q,
                     uint8_t* qs, int P, int K, hipStream_t st, const int32_t* x_rows = nullptr);
// mx_xform_in_q's rows as the fp8 operand: token p2u[r]'s codes and exponents copied to pair row r of qo / qso
// (equal to mx_xform_in_fp8 on the gathered rows).
void mx_xform_in_q_fp8(const uint8_t* q, const uint8_t* s, const int32_t* p2u, const MoePlan* plan,
                       const int32_t* row_expert, const uint8_t* const* s_tab, uint8_t* qo, uint8_t* qso, int P, int K,
                       hipStream_t st);
// mx_grouped_gemv / gemm / gemm_glu with the activations as (q, qs).
void mx_grouped_gemv_q(const uint8_t* q, const uint8_t* qs, int K, const Exl3Tile* tiles, int ntiles,
                       const uint8_t* const* w_tab, const uint8_t* const* s_tab, bf16* out, int ldo, int N,
                       hipStream_t st, const int* ntiles_dev = nullptr, const uint8_t* const* w_tab2 = nullptr,
                       const uint8_t* const* s_tab2 = nullptr, bf16* out2 = nullptr, int max_rows = kMxGemvTileRows,
                       const MxGlu& glu = {});
// mx_xform_in_fp8 + mx_grouped_gemv_q in one launch: each workgroup quantizes its tile's token rows x[x_rows[r]]
// (ldx apart; x_rows null: row r) per 128 exactly as act_quant_fp8 and keeps them in LDS. Bit-identical outputs.
void mx_grouped_gemv_x(const bf16* x, int ldx, const int32_t* x_rows, int K, const Exl3Tile* tiles, int ntiles,
                       const uint8_t* const* w_tab, const uint8_t* const* s_tab, bf16* out, int ldo, int N,
                       hipStream_t st, const int* ntiles_dev = nullptr, const uint8_t* const* w_tab2 = nullptr,
                       const uint8_t* const* s_tab2 = nullptr, bf16* out2 = nullptr, int max_rows = kMxGemvTileRows,
                       const MxGlu& glu = {});
// mx_xform_in_fp8 + mx_grouped_gemm_q in one launch (the workgroup quantizes its tile's token rows while staging).
void mx_grouped_gemm_x(const bf16* x, int ldx, const int32_t* x_rows, int K, const Exl3Tile* tiles, int ntiles,
                       const uint8_t* const* w_tab, const uint8_t* const* s_tab, bf16* out, int ldo, int N,
                       hipStream_t st, const int* ntiles_dev = nullptr, const uint8_t* const* w_tab2 = nullptr,
                       const uint8_t* const* s_tab2 = nullptr, bf16* out2 = nullptr, const MxGlu& glu = {});
// mx_grouped_gemm / mx_grouped_gemm_glu on bf16 rows gathered through x_rows: pair row r of a tile reads row
// x_rows[r] of xa ([rows, K] bf16; null: row r itself). No reference counterpart (the reference gathers the pair rows
// in mx_xform_in). K % 64, N % 128 (N % 256 without the epilogue).
void mx_grouped_gemm_rows(const bf16* xa, const int32_t* x_rows, int K, const Exl3Tile* tiles, int ntiles,
                          const uint8_t* const* w_tab, const uint8_t* const* s_tab, bf16* out, int ldo, int N,
                          hipStream_t st, const int* ntiles_dev = nullptr, const uint8_t* const* w_tab2 = nullptr,
                          const uint8_t* const* s_tab2 = nullptr, bf16* out2 = nullptr, const MxGlu& glu = {});
// The prefill GEMM on e4m3 codes with fp32 outputs (no bf16 rounding): for accuracy checks against an fp64 oracle.
// No reference counterpart.
void mx_grouped_gemm_q_f32out(const uint8_t* q, const uint8_t* qs, int K, const Exl3Tile* tiles, int ntiles,
                              const uint8_t* const* w_tab, const uint8_t* const* s_tab, float* out, int ldo, int N,
                              hipStream_t st, const int* ntiles_dev = nullptr);
// The arithmetic of the prefill GEMM on e4m3 codes (no reference counterpart): 1 (default) exact dequantization to
// bf16 + bf16 MFMA (fp32 sums of exact products, the reference's arithmetic in another order); 0 the block-scaled
// MFMA (fp8 x fp4 with the e8m0 scales in the instruction), a labelled speed mode outside the parity tolerance: its
// internal sums lose bits (~3e-3 of the output at the 2^-8 rms floor against fp64). UH_GEMM_EXACT=0 sets the
// default to 0. Returns the previous setting.
int mx_gemm_set_exact(int on);
bool mx_gemm_exact();
// The GEMV with fp32 outputs (no bf16 rounding): for accuracy checks against an fp64 oracle.
void mx_grouped_gemv_q_f32out(const uint8_t* q, const uint8_t* qs, int K, const Exl3Tile* tiles, int ntiles,
                              const uint8_t* const* w_tab, const uint8_t* const* s_tab, float* out, int ldo, int N,
                              hipStream_t st, const int* ntiles_dev = nullptr, int max_rows = kMxGemvTileRows);
// x_rows (optional): pair row r reads row x_rows[r] of q / qs (token rows quantized once, gathered by the loads).
void mx_grouped_gemm_q(const uint8_t* q, const uint8_t* qs, int K, const Exl3Tile* tiles, int ntiles,
                       const uint8_t* const* w_tab, const uint8_t* const* s_tab, bf16* out, int ldo, int N,
                       hipStream_t st, const int* ntiles_dev = nullptr, const uint8_t* const* w_tab2 = nullptr,
                       const uint8_t* const* s_tab2 = nullptr, bf16* out2 = nullptr, int max_rows = kExl3TileRows,
                       const MxGlu& glu = {}, const int32_t* x_rows = nullptr);

}  // namespace unholy::kernels
