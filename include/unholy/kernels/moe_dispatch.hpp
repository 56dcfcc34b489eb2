// Device-side MoE dispatch: routing bookkeeping between the router and the grouped expert kernels, with every
// routing-dependent size kept on the device (consumers launch for the maximum and read the real extents from
// MoePlan / ntiles_dev). Drop-in for src/kernels/moe_dispatch.hpp of the reference (single-device subset).
//
// The permutation is deterministic: rows of expert e are its tokens in ascending token order (the reference's
// host path, src/model/forward_ref.hip:1302-1328), computed with scans instead of the reference device path's
// atomic arrival order (moe_dispatch.hip:9-10). The combine follows pidx, so results never depend on it.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "unholy/kernels/elem_fast.hpp"

#include "unholy/kernels/exl3_moe.hpp"

namespace unholy::kernels {

struct MoePlan {  // ref moe_dispatch.hpp:14-20
  int P;
  int remote0;
  int n_local_tiles;
  int n_remote_tiles;
  int n_remote_tokens;
};

// count[e] += picks of e (count zero on entry; moe_plan clears it again); hist[e] += the same. Ref :26.
// Ref moe_dispatch.hpp:25: dst[i] = sel[i] as a byte, i < n (dst: pinned host memory; the routing trace).
void moe_trace(const int32_t* sel, int n, uint8_t* dst, hipStream_t st);
void moe_count(const int32_t* sel, int T, int K, int32_t* count, int E, hipStream_t st, uint32_t* hist = nullptr);
// Offsets (resident experts first, then the others, each ascending), tiles of <= tile_rows rows, plan; clears
// fill and count. resident may be null (all resident). E <= 1024. Ref :29-31.
void moe_plan(int32_t* count, const uint8_t* resident, int E, int P, MoePlan* plan, Exl3Tile* local_tiles,
              Exl3Tile* remote_tiles, int32_t* off, int32_t* fill, int max_tiles, hipStream_t st,
              int tile_rows = kExl3TileRows);
// Per token: its K picks sorted by expert id, pick j of token t -> pair row off[e] + (its rank among e's tokens).
// eidx[p] = token, ewt[p] = weight, row_expert[p] = e, pidx[t][j] = p. fill is not used. E is taken from the
// largest expert id present; the kernel scans sel per expert. Ref :32-33.
void moe_scatter(const int32_t* sel, const float* wt, int T, int K, const int32_t* off, int32_t* fill, int32_t* eidx,
                 float* ewt, int32_t* row_expert, int32_t* pidx, hipStream_t st);
// The same outputs as moe_scatter when the expert count is known (the kernel needs E; moe_scatter derives it).
void moe_scatter_e(const int32_t* sel, const float* wt, int T, int K, int E, const int32_t* off, int32_t* eidx,
                   float* ewt, int32_t* row_expert, int32_t* pidx, hipStream_t st);

// count + plan + scatter (optionally routing first) for steps of up to kMoeSmallMaxTokens tokens in one
// single-block launch. Ref :79-124. resident (null: all resident) puts the other experts' rows after remote0 and their
// tiles in rtl. With remote: stage_remote's outputs (plan_dst, tiles_dst, w_dst, e_dst); with qin also remote_tokens'
// (tok2u, u2t, p2u_dst, u2p_dst), and then x_dst (copy_remote_tokens) and q_dst / qs_dst (quant_remote_tokens) when
// given; req_flag: value stored with system-scope release after every write above.
constexpr int kMoeSmallMaxTokens = 32;
struct MoeSmallArgs {
  const int32_t* sel;
  const float* wt;
  int T, K;
  uint32_t* hist;
  const uint8_t* resident;
  int E, P, max_tiles, tile_rows;
  MoePlan* plan;
  Exl3Tile *lt, *rtl;
  int32_t* eidx;
  float* ewt;
  int32_t *row_expert, *pidx;
  bool remote, qin;
  int32_t *tok2u, *u2t, *p2u_dst, *u2p_dst;
  MoePlan* plan_dst;
  Exl3Tile* tiles_dst;
  float* w_dst;
  int32_t* e_dst;
  const float* route_logits = nullptr;  // GLM sigmoid routing in the launch
  const float* route_bias = nullptr;
  float route_scale = 0.0f;
  const uint16_t* x = nullptr;
  int dim = 0;
  uint16_t* x_dst = nullptr;
  const float* ds_logits = nullptr;  // DSV4 sqrt-softplus routing in the launch
  const float* ds_bias = nullptr;
  const float* ds_bias_vl = nullptr;
  const int32_t* ds_tid2eid = nullptr;
  const int32_t* ids = nullptr;
  int vocab = 0;
  uint8_t* q_dst = nullptr;
  uint8_t* qs_dst = nullptr;
  uint32_t* req_flag = nullptr;
  uint32_t req_value = 0;
  // Extension (no counterpart in the reference): softmax top-K routing in the launch (route_softmax's picks and
  // weights written to sel / wt).
  const float* softmax_logits = nullptr;
};
void moe_dispatch_small(const MoeSmallArgs& a, hipStream_t st);
// No reference counterpart: the same single-block launch for local steps of up to kMoeMidMaxPicks picks (T * K; no
// remote outputs, no resident mask), e.g. a 64-token verify step at top-6.
constexpr int kMoeMidMaxPicks = 512;
void moe_dispatch_mid(const MoeSmallArgs& a, hipStream_t st);

// ---- remote experts (the compact transport of experts held elsewhere) -------------------------------------------------
// Kernels with device-side extents (the plan); grids sized for max_rows / max_tokens. Each ends with a system-scope
// fence so a peer reading pinned host memory over the link sees its writes.
// Ref moe_dispatch.hpp:34-40: rows [remote0, P) of src -> the same rows of dst; the plan, remote tiles and the remote
// rows' routing weights and experts -> the remote side's staging.
void copy_remote_rows(const uint16_t* src, uint16_t* dst, const MoePlan* plan, int dim, int max_rows, hipStream_t st);
void stage_remote(const MoePlan* plan, const Exl3Tile* rtiles, const float* ewt, const int32_t* row_expert,
                  MoePlan* plan_dst, Exl3Tile* tiles_dst, float* w_dst, int32_t* e_dst, int max_rows, hipStream_t st);
// Ref moe_dispatch.hpp:125-126: the remote rows' weights and experts only.
void copy_remote_meta(const float* ewt, const int32_t* row_expert, float* w_dst, int32_t* e_dst, const MoePlan* plan,
                      int max_rows, hipStream_t st);
// Ref moe_dispatch.hpp:41-46: the tokens with at least one remote pair, in token order: tok2u [T] (-1: none),
// u2t [U], plan->n_remote_tokens = U, p2u_dst[p] = tok2u[eidx[p]] for p in [remote0, P), and with u2p_dst,
// u2p_dst[u * K + j] = token u's j-th pair row if remote, else -1. One workgroup.
void remote_tokens(const int32_t* pidx, const int32_t* eidx, int T, int K, MoePlan* plan, int32_t* tok2u,
                   int32_t* u2t, int32_t* p2u_dst, int32_t* u2p_dst, hipStream_t st);
// Ref moe_dispatch.hpp:47-52: dst[u] = bf16(sum over token u's remote pair rows of pair_out, fp32 adds in pick
// (ascending expert) order) for u < n_remote_tokens. dim % 8, 16-byte aligned rows.
void remote_combine(const uint16_t* pair_out, const int32_t* u2p, const MoePlan* plan, uint16_t* dst, int K, int dim,
                    int max_tokens, hipStream_t st);
// Ref moe_dispatch.hpp:53-57: dst[u] = x[u2t[u]] for u < n_remote_tokens.
void copy_remote_tokens(const uint16_t* x, int dim, const int32_t* u2t, const MoePlan* plan, uint16_t* dst,
                        int max_tokens, hipStream_t st);
// Ref moe_dispatch.hpp:58-60: src rows (remote_combine's dst) -> rows [remote0, remote0 + U) of dst.
void copy_remote_partial(const uint16_t* src, uint16_t* dst, const MoePlan* plan, int dim, int max_tokens,
                         hipStream_t st);
// Ref moe_dispatch.hpp:61-64: out[t] = bf16(token t's local pair rows (pidx order) + its remote partial row
// (pair_out row remote0 + tok2u[t]) + shared[t]), fp32 adds from 0 (shared null: no term).
void moe_combine_partial(const uint16_t* pair_out, const int32_t* pidx, const MoePlan* plan, const int32_t* tok2u,
                         const uint16_t* shared, uint16_t* out, int T, int K, int dim, hipStream_t st);
// Ref moe_dispatch.hpp:65-70: the same with the remote partial read from row tok2u[t] of `remote`; with hp.x, the
// mHC post-mix of each combined value into the token's streams.
void moe_combine_partial_link(const uint16_t* pair_out, const int32_t* pidx, const MoePlan* plan, const int32_t* tok2u,
                              const uint16_t* remote, const uint16_t* shared, uint16_t* out, int T, int K, int dim,
                              hipStream_t st, const HcPostArgs& hp = {});

// Ref moe_dispatch.hpp:71-76: act_quant_fp8 (block 128) of the rows x[u2t[u]] [dim] for u < plan->n_remote_tokens
// (a device-side count) into q_dst [U, dim] / s_dst [U, dim / 128]: the compact fp8 form of the tokens whose experts
// run on another device. Grid sized for max_tokens; dim % 128 == 0, x 16-byte aligned.
void quant_remote_tokens(const uint16_t* x, int dim, const int32_t* u2t, const MoePlan* plan, uint8_t* q_dst,
                         uint8_t* s_dst, int max_tokens, hipStream_t st);

}  // namespace unholy::kernels
