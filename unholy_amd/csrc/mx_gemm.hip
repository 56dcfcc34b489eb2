// Grouped GEMM for prefill tiles (rows > 16 per tile) and the dense fp8 GEMM dispatcher.
#include <algorithm>

#include "common.hpp"
#include "numerics.hpp"
#include "unholy/kernels/mx_moe.hpp"
#include "mx_internal.hpp"
#include "fp8_internal.hpp"

namespace unholy::kernels {

using namespace uh;

void launch_mx_gemm(const MxGemvArgs& a0, int ntiles, int amode, hipStream_t st) {
  MxGemvArgs a = a0;
  a.rows_cap = 16;
  launch_mx_gemv(a, ntiles, amode, st);
}

void launch_fp8_gemm(const Fp8GemmArgs& a, hipStream_t st) { launch_fp8_skinny(a, st); }

namespace {
MxGemvArgs gemm_args(const bf16* xa, const uint8_t* q, const uint8_t* qs, int K, const Exl3Tile* tiles,
                     const uint8_t* const* w_tab, const uint8_t* const* s_tab, bf16* out, int ldo, int N,
                     const int* ntiles_dev, const uint8_t* const* w_tab2, const uint8_t* const* s_tab2, bf16* out2,
                     const MxGlu& glu) {
  if (!w_tab || !s_tab) throw std::runtime_error("mx_grouped_gemm: null tables");
  if (!w_tab2 != !s_tab2) throw std::runtime_error("mx_grouped_gemm: second projection tables");
  MxGemvArgs a{};
  a.xa = xa;
  a.aq = q;
  a.as = qs;
  a.K = K;
  a.N = N;
  a.ldo = ldo;
  a.tiles = tiles;
  a.ntiles_dev = ntiles_dev;
  a.w_tab[0] = w_tab;
  a.s_tab[0] = s_tab;
  a.out[0] = out;
  a.w_tab[1] = w_tab2;
  a.s_tab[1] = s_tab2;
  a.out[1] = out2;
  a.gw = glu.w;
  a.grow_expert = glu.row_expert;
  a.gs_tab = glu.s_tab;
  a.hh = glu.hh;
  a.hq = glu.hq;
  a.hs = glu.hs;
  a.limit = glu.limit;
  if ((a.hh || a.hq) && a.gs_tab && !a.grow_expert) throw std::runtime_error("MxGlu: s_tab without row_expert");
  return a;
}
}  // namespace

void mx_grouped_gemm(const bf16* xa, int K, const Exl3Tile* tiles, int ntiles, const uint8_t* const* w_tab,
                     const uint8_t* const* s_tab, bf16* out, int ldo, int N, hipStream_t st, const int* ntiles_dev,
                     const uint8_t* const* w_tab2, const uint8_t* const* s_tab2, bf16* out2, int) {
  launch_mx_gemm(gemm_args(xa, nullptr, nullptr, K, tiles, w_tab, s_tab, out, ldo, N, ntiles_dev, w_tab2, s_tab2, out2,
                           MxGlu{}),
                 ntiles, 1, st);
}

void mx_grouped_gemm_q(const uint8_t* q, const uint8_t* qs, int K, const Exl3Tile* tiles, int ntiles,
                       const uint8_t* const* w_tab, const uint8_t* const* s_tab, bf16* out, int ldo, int N,
                       hipStream_t st, const int* ntiles_dev, const uint8_t* const* w_tab2,
                       const uint8_t* const* s_tab2, bf16* out2, int, const MxGlu& glu) {
  launch_mx_gemm(gemm_args(nullptr, q, qs, K, tiles, w_tab, s_tab, out, ldo, N, ntiles_dev, w_tab2, s_tab2, out2, glu),
                 ntiles, 0, st);
}

void mx_grouped_gemm_glu(const bf16* xa, int K, const Exl3Tile* tiles, int ntiles, const uint8_t* const* w1_tab,
                         const uint8_t* const* s1_tab, const uint8_t* const* w3_tab, const uint8_t* const* s3_tab, int N,
                         const MxGlu& glu, hipStream_t st, const int* ntiles_dev) {
  if (!glu.hh && !glu.hq) throw std::runtime_error("mx_grouped_gemm_glu: glu.hh");
  if (!glu.s_tab || !glu.row_expert) throw std::runtime_error("mx_grouped_gemm_glu: glu");
  launch_mx_gemm(gemm_args(xa, nullptr, nullptr, K, tiles, w1_tab, s1_tab, nullptr, N, N, ntiles_dev, w3_tab, s3_tab,
                           nullptr, glu),
                 ntiles, 1, st);
}

}  // namespace unholy::kernels
