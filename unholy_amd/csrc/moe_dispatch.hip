// Routing, dispatch bookkeeping, SwiGLU, gather/scatter and combine for the routed-expert path on gfx950.
// Interfaces: include/unholy/kernels/moe_dispatch.hpp and ref.hpp.
//
// The dispatch permutation is deterministic (rows of an expert = its tokens in ascending order, each token's
// picks sorted by expert id: src/model/forward_ref.hip:1302-1328): a block per expert walks the tokens in order
// and ranks its own picks with a block scan, instead of the reference device path's atomic fill counters
// (src/kernels/moe_dispatch.hip:82-109).
#include <algorithm>
#include <cmath>

#include "common.hpp"
#include "numerics.hpp"
#include "unholy/kernels/moe_dispatch.hpp"
#include "unholy/kernels/ref.hpp"
#include "mx_internal.hpp"

namespace unholy::kernels {

using namespace uh;

namespace {

constexpr int kMaxK = 8;

// Exclusive scan of v over a block of NT threads (NT / 64 waves); returns the prefix, total in *tot.
template <int NT>
__device__ __forceinline__ int block_exclusive_scan(int v, int* tot, int* lds /* >= NT/64 + 1 ints */) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int inc = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(inc, o, 64);
    if (lane >= o) inc += y;
  }
  if (lane == 63) lds[wave] = inc;
  __syncthreads();
  if (threadIdx.x == 0) {
    int run = 0;
    for (int w = 0; w < NT / 64; ++w) {
      const int c = lds[w];
      lds[w] = run;
      run += c;
    }
    lds[NT / 64] = run;
  }
  __syncthreads();
  const int res = lds[wave] + inc - v;
  *tot = lds[NT / 64];
  __syncthreads();
  return res;
}

__global__ void moe_count_kernel(const int32_t* __restrict__ sel, int n, int32_t* count, uint32_t* hist) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  atomicAdd(&count[sel[i]], 1);
  if (hist) atomicAdd(&hist[sel[i]], 1u);
}

// The same counts for E <= 1024: a histogram of CNT_PER picks in LDS per workgroup, then one global add per nonzero
// bin (integer sums: the result does not depend on the order). One global atomic per pick on a few hundred counters
// serialises at the counters.
constexpr int CNT_NT = 1024, CNT_PER = 4 * CNT_NT;
__global__ __launch_bounds__(CNT_NT) void moe_count_lds_kernel(const int32_t* __restrict__ sel, int n, int E,
                                                               int32_t* count, uint32_t* hist) {
  __shared__ int bins[1024];
  for (int e = threadIdx.x; e < E; e += CNT_NT) bins[e] = 0;
  __syncthreads();
  const int i0 = blockIdx.x * CNT_PER, i1 = min(n, i0 + CNT_PER);
  for (int i = i0 + threadIdx.x; i < i1; i += CNT_NT) atomicAdd(&bins[sel[i]], 1);
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += CNT_NT) {
    const int c = bins[e];
    if (!c) continue;
    atomicAdd(&count[e], c);
    if (hist) atomicAdd(&hist[e], uint32_t(c));
  }
}

// Offsets and tiles for E <= 1024 experts: resident experts first, then the others, each in ascending id
// (ref moe_dispatch.hip:39-79 semantics; scans here are wave shuffles plus one LDS pass).
constexpr int PLAN_NT = 1024;
__global__ __launch_bounds__(PLAN_NT) void moe_plan_kernel(int32_t* count, const uint8_t* resident, int E, int P,
                                                           MoePlan* plan, Exl3Tile* local_tiles,
                                                           Exl3Tile* remote_tiles, int32_t* off, int32_t* fill,
                                                           int max_tiles, int tile_rows) {
  __shared__ int lds[4][PLAN_NT / 64 + 1];
  const int e = threadIdx.x;
  const bool in = e < E, loc = in && (!resident || resident[e] != 0);
  const int c = in ? count[e] : 0, nt = (c + tile_rows - 1) / tile_rows;
  int tot[4];
  const int lrow = block_exclusive_scan<PLAN_NT>(loc ? c : 0, &tot[0], lds[0]);
  const int rrow = block_exclusive_scan<PLAN_NT>(in && !loc ? c : 0, &tot[1], lds[1]);
  const int ltile = block_exclusive_scan<PLAN_NT>(loc ? nt : 0, &tot[2], lds[2]);
  const int rtile = block_exclusive_scan<PLAN_NT>(in && !loc ? nt : 0, &tot[3], lds[3]);
  const int remote0 = tot[0];
  if (in) {
    const int row = loc ? lrow : remote0 + rrow, tile = loc ? ltile : rtile;
    Exl3Tile* dst = loc ? local_tiles : remote_tiles;
    off[e] = row;
    if (dst)
      for (int i = 0; i < nt && tile + i < max_tiles; ++i)
        dst[tile + i] = Exl3Tile{e, row + i * tile_rows, min(tile_rows, c - i * tile_rows)};
    if (fill) fill[e] = 0;
    count[e] = 0;
  }
  if (e == 0) {
    plan->P = P;
    plan->remote0 = remote0;
    plan->n_local_tiles = min(tot[2], max_tiles);
    plan->n_remote_tiles = min(tot[3], max_tiles);
    plan->n_remote_tokens = 0;
  }
}

// Block e: the tokens that picked e, in token order, get rows off[e], off[e] + 1, ...; each gets pidx at its
// position among its own picks sorted by expert id (the number of its picks below e; equal picks stay in
// selection order). A thread per token, SC_NT tokens per pass (one block scan); the next pass's picks are loaded
// before this pass's scan, so their latency overlaps it.
constexpr int SC_NT = 1024;
__global__ __launch_bounds__(SC_NT) void moe_scatter_kernel(const int32_t* __restrict__ sel, const float* __restrict__ wt,
                                                            int T, int K, const int32_t* __restrict__ off,
                                                            int32_t* eidx, float* ewt, int32_t* row_expert,
                                                            int32_t* pidx) {
  __shared__ int lds[SC_NT / 64 + 1];
  const int e = blockIdx.x;
  int run = 0, base_row = -1;
  int cur[kMaxK], nxt[kMaxK];
  const auto load = [&](int t, int (&v)[kMaxK]) {
#pragma unroll
    for (int j = 0; j < kMaxK; ++j) v[j] = (t < T && j < K) ? sel[size_t(t) * K + j] : -1;
  };
  load(threadIdx.x, cur);
  for (int t0 = 0; t0 < T; t0 += SC_NT) {
    const int t = t0 + threadIdx.x;
    load(t + SC_NT, nxt);
    int c = 0, below = 0;
#pragma unroll
    for (int j = 0; j < kMaxK; ++j) {
      c += cur[j] == e;
      below += cur[j] >= 0 && cur[j] < e;
    }
    int tot;
    const int pre = block_exclusive_scan<SC_NT>(c, &tot, lds);
    if (c) {
      if (base_row < 0) base_row = off[e];
      int d = 0;
#pragma unroll
      for (int j = 0; j < kMaxK; ++j)
        if (cur[j] == e) {
          const int p = base_row + run + pre + d;
          eidx[p] = t;
          ewt[p] = wt ? wt[size_t(t) * K + j] : 1.0f;
          row_expert[p] = e;
          pidx[size_t(t) * K + below + d] = p;
          ++d;
        }
    }
    run += tot;
#pragma unroll
    for (int j = 0; j < kMaxK; ++j) cur[j] = nxt[j];
  }
}

// ---- routers: a wave per token ---------------------------------------------------------------------------------------
__device__ __forceinline__ float ds_score(float x) { return sqrtf(x > 20.0f ? x : log1pf(expf(x))); }
__device__ __forceinline__ float sigmoid(float x) {
#pragma clang fp contract(off)
  return 1.0f / (1.0f + uh::exp_f32(-x));
}
__device__ __forceinline__ float lane_f32(float v, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l)); }

// One token's routing by one wave (MODE 0: DSV4 sqrt-softplus + bias or the hash row, 1: GLM sigmoid + bias, 2:
// softmax top-K; E <= 64 * NV). Lane l holds the keys of experts l + 64 i. Top-K with ties to the lower index, in
// selection order: per round the largest key (a DPP max of the order-preserving bits), then the lowest expert holding
// it (a DPP min); the pick's logit comes from the lane that holds it (readlane, no memory access). The picks are kept
// spread over lanes (lane k holds pick k) and every loop over them is a rolled loop over K: this code runs once per
// launch from a cold instruction cache, so its size sets its time more than its instruction count does.
// Weights (lane 0's order of operations in the reference's routers): GLM reports its picks in ascending id, the
// weights follow that order; mode 0 score / sum * scale, 1 sigmoid / (sum + 1e-20) * scale, 2 exp(l - l_first) / sum,
// the sum taken pick by pick from zero. Lanes k < K write pick k to sel_t / wt_t (and ssel / swt when set).
// pre (may be null): the lane's logits already loaded (pre[i] = lr[lane + 64 i], 0 past E).
template <int MODE, int NV>
__device__ __forceinline__ void route_wave(const float* lr, const float* bias, const int32_t* hash_row, int E, int K,
                                           float route_scale, int32_t* sel_t, float* wt_t, int* ssel, float* swt,
                                           const float* pre = nullptr) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  int pick = 0;
  float lgt = 0.0f;
  if (MODE == 0 && hash_row) {
    if (lane < K) {
      pick = hash_row[lane];
      lgt = lr[pick];
    }
  } else {
    float key[NV], raw[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int e = lane + 64 * i;
      raw[i] = pre ? pre[i] : e < E ? lr[e] : 0.0f;
      float v = -INFINITY;
      if (e < E) {
        if constexpr (MODE == 2) v = raw[i];
        else if constexpr (MODE == 1) v = sigmoid(raw[i]) + bias[e];
        else v = ds_score(raw[i]) + bias[e];
      }
      key[i] = v;
    }
    for (int k = 0; k < K; ++k) {
      float bv = -INFINITY;
      uint32_t bi = 0xffffffffu;
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int e = lane + 64 * i;
        if (e < E && (key[i] > bv || bi == 0xffffffffu)) bv = key[i], bi = uint32_t(e);
      }
      const uint32_t ob = bi == 0xffffffffu ? 0u : orderable(bv);
      const uint32_t m = wave_reduce_u32<true>(ob);
      // The lowest expert holding the largest key: when one lane holds it (the usual case) that lane's candidate,
      // else the DPP min over the lanes that do.
      const uint64_t holders = __ballot(ob == m);
      const uint32_t idx = __popcll(holders) == 1
                               ? uint32_t(__builtin_amdgcn_readlane(int(bi), int(__builtin_ctzll(holders))))
                               : wave_reduce_u32<false>(ob == m ? bi : 0xffffffffu);
      const int slot = int(idx >> 6), owner = int(idx & 63);
      float v = 0.0f;
#pragma unroll
      for (int i = 0; i < NV; ++i)
        if (slot == i) {
          v = raw[i];
          if (lane == owner) key[i] = -INFINITY;
        }
      const float l = lane_f32(v, owner);
      if (lane == k) pick = int(idx), lgt = l;
    }
  }
  if constexpr (MODE == 1) {  // ascending id: lane k's pick moves to lane (number of smaller picks)
    int r = lane;
    if (lane < K) {
      r = 0;
      for (int q = 0; q < K; ++q) r += __builtin_amdgcn_readlane(pick, q) < pick;
    }
    pick = __builtin_amdgcn_ds_permute(r * 4, pick);
    lgt = __int_as_float(__builtin_amdgcn_ds_permute(r * 4, __float_as_int(lgt)));
  }
  const float w = MODE == 2 ? uh::exp_f32(lgt - lane_f32(lgt, 0)) : MODE == 1 ? sigmoid(lgt) : ds_score(lgt);
  float sum = 0.0f;
  for (int k = 0; k < K; ++k) sum += lane_f32(w, k);
  if (lane < K) {
    const float wk = MODE == 2 ? w / sum : MODE == 1 ? w / (sum + 1e-20f) * route_scale : (w / sum) * route_scale;
    sel_t[lane] = pick;
    wt_t[lane] = wk;
    if (ssel) {
      ssel[lane] = pick;
      swt[lane] = wk;
    }
  }
}

// mode 0: DSV4 (sqrt-softplus + bias, hash tid2eid, bias_vl for image ids), 1: GLM sigmoid, 2: softmax top-K.
template <int MODE>
__global__ __launch_bounds__(256) void route_wave_kernel(const float* __restrict__ logits, const float* bias0,
                                                         const int32_t* tid2eid0, const int32_t* ids, int32_t* sel,
                                                         float* weights, int T, int E, int K, float route_scale,
                                                         const float* bias_vl, int vocab) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const bool image = MODE == 0 && bias_vl && ids[t] >= vocab;
  const float* bias = image ? bias_vl : bias0;
  const int32_t* hash_row = MODE == 0 && !image && tid2eid0 ? tid2eid0 + size_t(ids[t]) * K : nullptr;
  route_wave<MODE, 16>(logits + size_t(t) * E, bias, hash_row, E, K, route_scale, sel + size_t(t) * K,
                       weights + size_t(t) * K, nullptr, nullptr);
}

// The reference's one-thread-per-token DSV4 router (ref_moe.hip:14-60): the same picks and weights as the wave
// form; kept as the `route` entry point.
__global__ void route_thread_kernel(const float* logits, const float* bias0, const int32_t* tid2eid0,
                                    const int32_t* ids, int32_t* sel, float* weights, int T, int E, int K,
                                    float route_scale, const float* bias_vl, int vocab) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= T) return;
  const bool image = bias_vl && ids[t] >= vocab;
  const float* bias = image ? bias_vl : bias0;
  const int32_t* tid2eid = image ? nullptr : tid2eid0;
  const float* lg = logits + size_t(t) * E;
  int chosen[kMaxK];
  if (tid2eid) {
    for (int k = 0; k < K; ++k) chosen[k] = tid2eid[size_t(ids[t]) * K + k];
  } else {
    for (int k = 0; k < K; ++k) {
      int best = -1;
      float bv = -INFINITY;
      for (int e = 0; e < E; ++e) {
        bool used = false;
        for (int j = 0; j < k; ++j) used |= chosen[j] == e;
        if (used) continue;
        const float v = ds_score(lg[e]) + bias[e];
        if (best < 0 || v > bv) best = e, bv = v;
      }
      chosen[k] = best;
    }
  }
  float w[kMaxK], sum = 0.0f;
  for (int k = 0; k < K; ++k) {
    w[k] = ds_score(lg[chosen[k]]);
    sum += w[k];
  }
  for (int k = 0; k < K; ++k) {
    sel[size_t(t) * K + k] = chosen[k];
    weights[size_t(t) * K + k] = (w[k] / sum) * route_scale;
  }
}

// One token's routing by one wave inside moe_dispatch_small (MODE 0 DSV4, 1 GLM, 2 softmax; E <= 64 * NV).
template <int MODE>
__device__ __forceinline__ const float* route_row(const MoeSmallArgs& a, int t) {
  return (MODE == 2 ? a.softmax_logits : MODE == 1 ? a.route_logits : a.ds_logits) + size_t(t) * a.E;
}
template <int MODE, int NV>
__device__ __forceinline__ void route_token(const MoeSmallArgs& a, int t, int* skey, float* swt,
                                            const float* pre = nullptr) {
  const float* lr = route_row<MODE>(a, t);
  const bool image = MODE == 0 && a.ds_bias_vl && a.ids[t] >= a.vocab;
  const float* bias = MODE == 1 ? a.route_bias : image ? a.ds_bias_vl : a.ds_bias;
  const int32_t* hash_row = MODE == 0 && !image && a.ds_tid2eid ? a.ds_tid2eid + size_t(a.ids[t]) * a.K : nullptr;
  route_wave<MODE, NV>(lr, bias, hash_row, a.E, a.K, a.route_scale, const_cast<int32_t*>(a.sel) + size_t(t) * a.K,
                       const_cast<float*>(a.wt) + size_t(t) * a.K, skey + t * a.K, swt + t * a.K, pre);
}
// A wave's tokens t = first, first + stride, ...: the next token's logits are loaded before this one is routed.
template <int MODE, int NV>
__device__ __forceinline__ void route_tokens(const MoeSmallArgs& a, int first, int stride, int* skey, float* swt) {
  const int lane = threadIdx.x & 63;
  const auto load = [&](int t, float (&v)[NV]) {
    const float* lr = route_row<MODE>(a, t);
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] = lane + 64 * i < a.E ? lr[lane + 64 * i] : 0.0f;
  };
  float nxt[NV];
  if (first < a.T) load(first, nxt);
  for (int t = first; t < a.T; t += stride) {
    float cur[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) cur[i] = nxt[i];
    if (t + stride < a.T) load(t + stride, nxt);
    route_token<MODE, NV>(a, t, skey, swt, cur);
  }
}

// ---- single-block dispatch for small steps -------------------------------------------------------------------------
// T <= 32 tokens, K <= 8 picks: n = T * K <= 256 pair rows, one thread per pick. Optional routing first (a wave per
// token). Pick i = t * K + j gets the key (e * T + t) * K + j; its pair row is the number of smaller keys, which is
// exactly the host order (experts ascending, tokens ascending within an expert, equal picks of one token in
// selection order); the same counting pass gives the expert's first row (keys of smaller experts) and its row
// count. Tiles start where a row is a multiple of tile_rows into its expert's run; their index is a block scan.
constexpr int SMALL_NT = 512;
__global__ __launch_bounds__(SMALL_NT) void moe_dispatch_small_kernel(MoeSmallArgs a) {
  __shared__ __align__(16) int skey[SMALL_NT];
  __shared__ float swt[SMALL_NT];
  __shared__ int lds[SMALL_NT / 64 + 1];
  const int T = a.T, K = a.K, E = a.E, n = T * K, tid = threadIdx.x, wave = tid >> 6;
  // The arguments every launch uses, read into scalar registers here: one wait for all of them, instead of a
  // scalar-cache miss at each first use further down (a kernel-argument line is not cached from the last launch).
  asm volatile("" ::"s"(a.softmax_logits), "s"(a.route_logits), "s"(a.ds_logits), "s"(a.eidx), "s"(a.ewt),
               "s"(a.row_expert), "s"(a.pidx), "s"(a.lt), "s"(a.plan), "s"(a.tile_rows), "s"(a.max_tiles),
               "s"(a.resident), "s"(a.hist), "s"(a.P), "s"(a.sel), "s"(a.wt));
  // Steps with more picks than one wave and no resident mask rank their picks by expert counts (histogram +
  // scan) instead of comparing every pair of keys; the counts are cleared here, while the routing loads are out.
  const bool by_hist = n > 64 && !a.resident;
  __shared__ int ehist[1024], wcnt[SMALL_NT / 64][1024];  // picks per expert; per wave
  if (by_hist)
    for (int q = tid; q < (SMALL_NT / 64 + 1) * E; q += SMALL_NT) {
      if (q < E) ehist[q] = 0;
      else wcnt[q / E - 1][q % E] = 0;
    }
  const bool route = a.route_logits || a.ds_logits || a.softmax_logits;
  if (route) {
    const int mode = a.softmax_logits ? 2 : a.route_logits ? 1 : 0;
    constexpr int S = SMALL_NT / 64;
    if (E <= 256) {
      if (mode == 2) route_tokens<2, 4>(a, wave, S, skey, swt);
      else if (mode == 1) route_tokens<1, 4>(a, wave, S, skey, swt);
      else route_tokens<0, 4>(a, wave, S, skey, swt);
    } else {
      if (mode == 2) route_tokens<2, 16>(a, wave, S, skey, swt);
      else if (mode == 1) route_tokens<1, 16>(a, wave, S, skey, swt);
      else route_tokens<0, 16>(a, wave, S, skey, swt);
    }
  } else {
    for (int i = tid; i < n; i += SMALL_NT) {
      skey[i] = a.sel[i];
      swt[i] = a.wt[i];
    }
  }
  __syncthreads();
  if (n <= 64 && !a.remote && !a.resident && !a.hist) {
    // The forward's decode case (all picks fit one wave, only the local plan is asked for): wave 0 alone finishes
    // the dispatch with no further barrier. Lane l stands for pick l (token l / K, selection l % K). The expert's
    // bits are walked from the top with ballots: `less` collects the picks whose expert is smaller, `peers` ends as
    // the picks of the same expert. Within an expert the plan orders rows by (token, selection), which is the pick
    // index order, so pair row p = |less| + (peers below this lane); token t's picks before this one by (expert,
    // selection) are the same counts restricted to the token's K lanes.
    if (wave != 0) return;
    const int l = tid;
    const bool live = l < n;
    const int e = live ? skey[l] : 0;
    const float w = live ? swt[l] : 0.0f;
    const int t = live ? l / K : 0;
    uint64_t peers = __ballot(live), less = 0;
    for (int b = 31 - __builtin_clz(uint32_t(max(E - 1, 1))); b >= 0; --b) {
      const uint64_t ones = __ballot(live && ((e >> b) & 1));
      if ((e >> b) & 1) {
        less |= peers & ~ones;
        peers &= ones;
      } else {
        peers &= ~ones;
      }
    }
    const auto below_me = [](uint64_t m) {
      return int(__builtin_amdgcn_mbcnt_hi(uint32_t(m >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(m), 0u)));
    };
    const uint64_t tok = ((K >= 64 ? ~0ull : (1ull << K) - 1)) << (t * K);
    const int off = __popcll(less), cnt = __popcll(peers), p = off + below_me(peers);
    const int below = __popcll(less & tok) + below_me(peers & tok);
    __shared__ int sflag[64], srow_e1[64], sleft[64];  // per pair row
    if (live) {
      a.eidx[p] = t;
      a.ewt[p] = w;
      a.row_expert[p] = e;
      a.pidx[size_t(t) * K + below] = p;
      // rows of the expert's run from here when this row starts a tile (a multiple of tile_rows into the run)
      sflag[p] = (p - off) % a.tile_rows == 0;
      srow_e1[p] = e;
      sleft[p] = cnt - (p - off);
    }
    __builtin_amdgcn_wave_barrier();  // one wave: its LDS accesses complete in order
    // Lane r now stands for pair row r: tiles are numbered in row order (a ballot prefix count).
    const int r = tid;
    const bool start = r < n && sflag[r];
    const uint64_t starts = __ballot(start);
    const int tile = below_me(starts);
    if (start && tile < a.max_tiles) a.lt[tile] = Exl3Tile{srow_e1[r], r, min(a.tile_rows, sleft[r])};
    if (tid == 0) *a.plan = MoePlan{a.P, n, min(int(__popcll(starts)), a.max_tiles), 0, 0};
    return;
  }
  const int i = tid;
  const bool live = i < n;
  int e = 0, t = 0, j = 0;
  float w = 0.0f;
  if (live) {
    e = skey[i];
    w = swt[i];
    t = i / K;
    j = i % K;
    if (a.hist) atomicAdd(&a.hist[e], 1u);
  }
  // Non-resident experts sort after every resident one: key class ek = e + E (resident first, then the others, each
  // in ascending id: the reference's plan order). Rows below remote0 = keys below E * T * K.
  const int ek = (a.resident && live && !a.resident[e]) ? e + E : e;
  __shared__ int sexp[SMALL_NT], sek[SMALL_NT];  // pick i's expert id and key class
  __syncthreads();
  if (live) {
    skey[i] = (ek * T + t) * K + j;
    sexp[i] = e;
    sek[i] = ek;
  }
  __syncthreads();
  const int mykey = (ek * T + t) * K + j, lo = ek * T * K, hi = (ek + 1) * T * K, lim = E * T * K;
  int rank = 0, off = 0, cnt = 0, nloc = 0;
  if (by_hist) {
    // Each wave groups its lanes by expert with a ballot walk over the expert's bits; the lowest lane of a group
    // records the group's size for its wave and adds it to the expert's count. An exclusive scan of the counts gives
    // each expert's first row; a pick's row adds the same expert's picks in earlier waves and in lower lanes (the
    // plan's order within an expert is the pick order). Every pick is resident: nloc = n.
    uint64_t peers = __ballot(live);
    for (int b = 31 - __builtin_clz(uint32_t(max(E - 1, 1))); b >= 0; --b) {
      const uint64_t ones = __ballot(live && ((e >> b) & 1));
      peers &= ((e >> b) & 1) ? ones : ~ones;
    }
    const int inwave = int(__builtin_amdgcn_mbcnt_hi(uint32_t(peers >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(peers), 0u)));
    if (live && inwave == 0) {
      wcnt[wave][e] = __popcll(peers);
      atomicAdd(&ehist[e], __popcll(peers));
    }
    __syncthreads();
    // exclusive scan over experts, two per thread (E <= 1024)
    const int e0 = 2 * tid, c0 = e0 < E ? ehist[e0] : 0, c1 = e0 + 1 < E ? ehist[e0 + 1] : 0;
    int total;
    const int ex = block_exclusive_scan<SMALL_NT>(c0 + c1, &total, lds);
    __shared__ int estart[1024];
    if (e0 < E) estart[e0] = ex;
    if (e0 + 1 < E) estart[e0 + 1] = ex + c0;
    __syncthreads();
    if (live) {
      off = estart[e];
      cnt = ehist[e];
      rank = off + inwave;
      for (int w = 0; w < wave; ++w) rank += wcnt[w][e];
      nloc = n;
    }
  } else if (n <= 64) {
    // All 8 waves count: wave w compares keys 8w .. 8w + 7 against pick l (lane l) and the partial counts are added
    // through LDS (an eighth of the serial compares of one wave doing all of them).
    __shared__ int4 spart[SMALL_NT / 64][64];
    const int l = tid & 63;
    int4 c = {0, 0, 0, 0};
    if (l < n) {
      const int mk = skey[l], lo_l = sek[l] * T * K, hi_l = lo_l + T * K;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int q = wave * 8 + u;
        if (q < n) {
          const int kq = skey[q];
          c.x += kq < mk;
          c.y += kq < lo_l;
          c.z += kq >= lo_l && kq < hi_l;
          c.w += kq < lim;
        }
      }
    }
    spart[wave][l] = c;
    __syncthreads();
    if (live)
#pragma unroll
      for (int w = 0; w < SMALL_NT / 64; ++w) {
        const int4 v = spart[w][tid];
        rank += v.x;
        off += v.y;
        cnt += v.z;
        nloc += v.w;
      }
  } else if (live) {
    int q = 0;
    // The same address in every lane: broadcast reads, sixteen keys (four 16-byte reads issued together) at a time.
    for (; q + 16 <= n; q += 16) {
      int4 k4[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) k4[v] = *reinterpret_cast<const int4*>(&skey[q + 4 * v]);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int kk[4] = {k4[v].x, k4[v].y, k4[v].z, k4[v].w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          rank += kk[u] < mykey;
          off += kk[u] < lo;
          cnt += kk[u] >= lo && kk[u] < hi;
          nloc += kk[u] < lim;
        }
      }
    }
    for (; q < n; ++q) {
      const int kq = skey[q];
      rank += kq < mykey;
      off += kq < lo;
      cnt += kq >= lo && kq < hi;
      nloc += kq < lim;
    }
  }
  const int remote0 = live ? nloc : 0;  // the same in every live thread; thread 0 is live (n >= 1)
  // Token t's picks ordered before this one by expert id, then selection order (the reference's sorted picks):
  int below = 0;
  if (live)
    for (int q = 0; q < K; ++q) {
      const int eq = sexp[t * K + q];
      below += eq < e || (eq == e && q < j);
    }
  const int p = rank;
  __shared__ int srow_e[SMALL_NT], srow_left[SMALL_NT], spidx[SMALL_NT];
  __shared__ int stok[kMoeSmallMaxTokens], su2t[kMoeSmallMaxTokens], sU;
  if (live) {
    a.eidx[p] = t;
    a.ewt[p] = w;
    a.row_expert[p] = e;
    a.pidx[size_t(t) * K + below] = p;
    spidx[t * K + below] = p;
    if (a.remote && p >= remote0) {  // stage_remote: the remote rows' weights and experts
      a.w_dst[p] = w;
      a.e_dst[p] = e;
    }
    srow_e[p] = e;
    // rows of the expert's run from here, or 0 when this row does not start a tile
    srow_left[p] = (p - off) % a.tile_rows == 0 ? cnt - (p - off) : 0;
  }
  __syncthreads();
  // Now thread r stands for pair row r: tiles are numbered in row order.
  const int r = tid, left = r < n ? srow_left[r] : 0;
  // Local and remote tile starts counted in one scan: the low half-word counts local ones, the high one remote ones
  // (at most 256 rows each). Local rows precede remote rows, so both numberings are in row order.
  int ntiles;
  const int tile = block_exclusive_scan<SMALL_NT>(left > 0 ? (r < remote0 ? 1 : 1 << 16) : 0, &ntiles, lds);
  if (left > 0) {
    const Exl3Tile tl{srow_e[r], r, min(a.tile_rows, left)};
    if (r < remote0) {
      if ((tile & 0xffff) < a.max_tiles) a.lt[tile & 0xffff] = tl;
    } else if ((tile >> 16) < a.max_tiles) {
      a.rtl[tile >> 16] = tl;
      if (a.remote) a.tiles_dst[tile >> 16] = tl;  // stage_remote: the remote tiles
    }
  }
  __shared__ int srem0;
  if (tid == 0) srem0 = remote0;
  // remote_tokens (moe_dispatch.hip:149-203) for T <= 32: token t has a remote pair when one of its rows is
  // >= remote0; those tokens, in order, get compact indices.
  if (a.remote && a.qin && tid < T) {
    bool f = false;
    for (int q = 0; q < K; ++q) f = f || skey[tid * K + q] >= lim;
    stok[tid] = f ? 1 : 0;
  }
  __syncthreads();
  const int R0 = srem0;
  if (a.remote && a.qin) {
    if (tid < T) {
      int ex = 0;
      for (int q = 0; q < tid; ++q) ex += stok[q];
      const bool f = stok[tid] != 0;
      a.tok2u[tid] = f ? ex : -1;
      if (f) {
        a.u2t[ex] = tid;
        su2t[ex] = tid;
        if (a.u2p_dst)
          for (int q = 0; q < K; ++q) {
            const int pq = spidx[tid * K + q];
            a.u2p_dst[size_t(ex) * K + q] = pq >= R0 ? pq : -1;
          }
      }
      if (tid == T - 1) sU = ex + (f ? 1 : 0);
    }
    if (live && p >= R0) {  // stok still holds the flags  // p2u[p] = the compact index of row p's token
      int ex = 0;
      for (int q = 0; q < t; ++q) ex += stok[q];
      a.p2u_dst[p] = ex;
    }
  } else if (tid == 0) {
    sU = 0;
  }
  __syncthreads();
  const int U = sU;
  const MoePlan pl{a.P, R0, min(ntiles & 0xffff, a.max_tiles), min(ntiles >> 16, a.max_tiles), U};
  if (tid == 0) {
    *a.plan = pl;
    if (a.remote) *a.plan_dst = pl;  // stage_remote: the plan
  }
  if (!a.remote) return;
  if (a.x_dst) {  // copy_remote_tokens: the remote tokens' rows of x, 16 bytes per thread
    const int cols = a.dim / 8;
    for (int i2 = tid; i2 < U * cols; i2 += SMALL_NT) {
      const int u = i2 / cols, c = i2 % cols;
      reinterpret_cast<uint4*>(a.x_dst + size_t(u) * a.dim)[c] =
          reinterpret_cast<const uint4*>(a.x + size_t(su2t[u]) * a.dim)[c];
    }
  }
  if (a.q_dst) {  // quant_remote_tokens: the same rows as e4m3 codes + e8m0 exponents
    const size_t items = size_t(U) * (a.dim / 8);
    for (size_t base = 0; base < items; base += SMALL_NT)
      quant_token_item(a.x, a.dim, su2t, a.q_dst, a.qs_dst, base + tid, items);
  }
  // One system-scope release, by wave 0 after the barrier (cumulative over it), then the request flag from the same
  // wave, so the flag is seen only after every write above.
  __syncthreads();
  if (tid < 64) {
    __threadfence_system();
    if (a.req_flag && tid == 0) __hip_atomic_store(a.req_flag, a.req_value, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

// ---- elementwise -----------------------------------------------------------------------------------------------------
__global__ void swiglu_kernel(const bf16* gate, const bf16* up, const float* w, bf16* h, int rows, int dim,
                              float limit) {
  const size_t gid = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (gid >= size_t(rows) * dim) return;
  h[gid] = f32_to_bf16(swiglu_value(bf16_to_f32(gate[gid]), bf16_to_f32(up[gid]), w ? w[gid / dim] : 0.0f,
                                    w != nullptr, limit));
}

__global__ void gather_rows_kernel(const bf16* src, const int32_t* rows_idx, bf16* dst, int n, int dim) {
  const size_t gid = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (gid >= size_t(n) * dim) return;
  dst[gid] = src[size_t(rows_idx[gid / dim]) * dim + gid % dim];
}

// One thread per column, rows in order (the same fp32 sums as the reference's row-ordered scatter).
__global__ void scatter_add_kernel(const bf16* src, const int32_t* rows_idx, float* y, int n, int dim) {
  const int d = blockIdx.x * blockDim.x + threadIdx.x;
  if (d >= dim) return;
  for (int r = 0; r < n; ++r) y[size_t(rows_idx[r]) * dim + d] += bf16_to_f32(src[size_t(r) * dim + d]);
}

// out[t][d] = bf16(sum_j pair_out[pidx[t][j]][d] (j ascending) + shared[t][d]): a thread per 8 columns.
__global__ __launch_bounds__(256) void moe_combine_kernel(const bf16* __restrict__ pair_out,
                                                          const int32_t* __restrict__ pidx,
                                                          const bf16* __restrict__ shared, bf16* __restrict__ out,
                                                          int K, int dim) {
  const int t = blockIdx.y, d = (blockIdx.x * 256 + threadIdx.x) * 8;
  if (d >= dim) return;
  float acc[8] = {};
  const auto add = [&](const uint4 v) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      acc[2 * q] += __uint_as_float(w[q] << 16);
      acc[2 * q + 1] += __uint_as_float(w[q] & 0xffff0000u);
    }
  };
  // Up to kMaxK picks: every row load is issued before the first add (one memory latency, not one per pick); the
  // adds stay in pick order.
  const int kk = min(K, kMaxK);
  uint4 v[kMaxK];
#pragma unroll
  for (int j = 0; j < kMaxK; ++j)
    if (j < kk) v[j] = *reinterpret_cast<const uint4*>(pair_out + size_t(pidx[size_t(t) * K + j]) * dim + d);
  const uint4 sv = shared ? *reinterpret_cast<const uint4*>(shared + size_t(t) * dim + d) : uint4{};
#pragma unroll
  for (int j = 0; j < kMaxK; ++j)
    if (j < kk) add(v[j]);
  for (int j = kMaxK; j < K; ++j) add(*reinterpret_cast<const uint4*>(pair_out + size_t(pidx[size_t(t) * K + j]) * dim + d));
  if (shared) {
    add(sv);
  } else {
#pragma unroll
    for (int q = 0; q < 8; ++q) acc[q] += 0.0f;
  }
  uint32_t o[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) o[q] = uint32_t(f32_to_bf16(acc[2 * q])) | uint32_t(f32_to_bf16(acc[2 * q + 1])) << 16;
  *reinterpret_cast<uint4*>(out + size_t(t) * dim + d) = make_uint4(o[0], o[1], o[2], o[3]);
}

// moe_trace (moe_dispatch.hpp:25): dst[i] = sel[i] as a byte, the routing trace written to pinned host memory.
__global__ __launch_bounds__(256) void moe_trace_kernel(const int32_t* __restrict__ sel, int n, uint8_t* __restrict__ dst) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) dst[i] = uint8_t(sel[i]);
}

// ---- remote experts: staging, compact tokens, partial combines (moe_dispatch.hip:111-278) ---------------------------
// Device-side extents (plan) with grids sized for the maximum: grid-stride loops over 16-byte units. Each kernel ends
// with a system-scope release so a host or peer reader of pinned memory sees its writes; one wave per workgroup runs
// it after a barrier (release is cumulative over the barrier), since each run waits on an L2 write-back.
__device__ __forceinline__ void fence_system_once() {
  __syncthreads();
  if (threadIdx.x < 64) __threadfence_system();
}
__global__ __launch_bounds__(256) void copy_rows16_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst,
                                                          const MoePlan* __restrict__ plan, int units_per_row,
                                                          int mode) {
  // mode 0: rows [remote0, P) to the same rows; 1: n_remote_tokens rows from src to rows remote0.. of dst
  const MoePlan pl = *plan;
  const size_t r0 = size_t(pl.remote0) * units_per_row;
  const size_t n = size_t(mode == 0 ? pl.P - pl.remote0 : pl.n_remote_tokens) * units_per_row;
  const uint4* s = mode == 0 ? src + r0 : src;
  uint4* o = dst + r0;
  for (size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x)
    o[i] = s[i];
  fence_system_once();
}

__global__ __launch_bounds__(256) void stage_remote_kernel(const MoePlan* __restrict__ plan,
                                                           const Exl3Tile* __restrict__ rtiles,
                                                           const float* __restrict__ ewt,
                                                           const int32_t* __restrict__ row_expert,
                                                           MoePlan* __restrict__ plan_dst,
                                                           Exl3Tile* __restrict__ tiles_dst, float* __restrict__ w_dst,
                                                           int32_t* __restrict__ e_dst, bool with_plan) {
  const MoePlan pl = *plan;
  const int tid = blockIdx.x * blockDim.x + threadIdx.x, nt = gridDim.x * blockDim.x;
  if (with_plan) {
    if (tid == 0) *plan_dst = pl;
    for (int i = tid; i < pl.n_remote_tiles; i += nt) tiles_dst[i] = rtiles[i];
  }
  for (int i = pl.remote0 + tid; i < pl.P; i += nt) {
    w_dst[i] = ewt[i];
    e_dst[i] = row_expert[i];
  }
  fence_system_once();
}

// One workgroup: an exclusive scan of "has a remote pair" over the tokens, 1024 at a time, then p2u over the remote
// rows (tok2u is read back after the barrier that ends the scan; this workgroup wrote it).
constexpr int RT_NT = 1024;
__global__ __launch_bounds__(RT_NT) void remote_tokens_kernel(const int32_t* __restrict__ pidx,
                                                              const int32_t* __restrict__ eidx, int T, int K,
                                                              MoePlan* __restrict__ plan, int32_t* __restrict__ tok2u,
                                                              int32_t* __restrict__ u2t, int32_t* __restrict__ p2u,
                                                              int32_t* __restrict__ u2p) {
  __shared__ int lds[RT_NT / 64 + 1];
  const int r0 = plan->remote0, P = plan->P, tid = threadIdx.x;
  int carry = 0;
  for (int base = 0; base < T; base += RT_NT) {
    const int t = base + tid;
    bool f = false;
    if (t < T)
      for (int j = 0; j < K; ++j) f = f || pidx[size_t(t) * K + j] >= r0;
    int tot;
    const int u = carry + block_exclusive_scan<RT_NT>(f ? 1 : 0, &tot, lds);
    if (t < T) {
      tok2u[t] = f ? u : -1;
      if (f) {
        u2t[u] = t;
        if (u2p)
          for (int j = 0; j < K; ++j) {
            const int p = pidx[size_t(t) * K + j];
            u2p[size_t(u) * K + j] = p >= r0 ? p : -1;
          }
      }
    }
    carry += tot;
  }
  __syncthreads();
  if (tid == 0) plan->n_remote_tokens = carry;
  for (int p = r0 + tid; p < P; p += RT_NT) p2u[p] = tok2u[eidx[p]];
  fence_system_once();
}

__device__ __forceinline__ void add_bf16x8(float (&acc)[8], const bf16* p) {
  const uint4 v = *reinterpret_cast<const uint4*>(p);
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    acc[2 * q] += __uint_as_float(w[q] << 16);
    acc[2 * q + 1] += __uint_as_float(w[q] & 0xffff0000u);
  }
}
__device__ __forceinline__ uint4 pack_bf16x8(const float (&acc)[8]) {
  uint32_t o[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) o[q] = uint32_t(f32_to_bf16(acc[2 * q])) | uint32_t(f32_to_bf16(acc[2 * q + 1])) << 16;
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// dst[u] = bf16(sum of token u's remote pair rows, fp32 adds from 0 in pick order): workgroup (2048-column chunk,
// token stride), a thread per 8 columns. The closing system-scope fence costs a write-back wait per wave that runs
// it, so one wave per workgroup runs it and the grid stays small (at most 256 token rows of workgroups, each striding
// over the compact tokens); rows are stored nontemporal (streamed past the cache).
__global__ __launch_bounds__(256) void remote_combine_kernel(const bf16* __restrict__ pair_out,
                                                             const int32_t* __restrict__ u2p,
                                                             const MoePlan* __restrict__ plan, bf16* __restrict__ dst,
                                                             int K, int dim, int ld) {
  const int d = (blockIdx.x * 256 + threadIdx.x) * 8, U = plan->n_remote_tokens;
  for (int u = blockIdx.y; u < U && d < dim; u += gridDim.y) {
    float acc[8] = {};
    for (int j = 0; j < K; ++j) {
      const int p = u2p[size_t(u) * K + j];
      if (p >= 0) add_bf16x8(acc, pair_out + size_t(p) * ld + d);
    }
    const uint4 o = pack_bf16x8(acc);
    using u32x4 = unsigned int __attribute__((ext_vector_type(4)));
    __builtin_nontemporal_store(u32x4{o.x, o.y, o.z, o.w}, reinterpret_cast<u32x4*>(dst + size_t(u) * dim + d));
  }
  fence_system_once();
}

// out[t] = bf16(local pair rows (p < remote0, pick order) + the token's remote row + shared[t]), fp32 adds from 0;
// remote null: the remote rows are pair_out's rows from remote0 on. With hp.x: the mHC post-mix of each output value
// into the token's hc streams in place, x[t][j][d] = bf16(fma(post[t][j], o, sum_i comb[t][i][j] * x[t][i][d])),
// the sum an fma chain over i (dev.hip.hpp:185-201). V = 8: 16-byte loads and stores; V = 1: one column.
template <int V>
__global__ __launch_bounds__(256) void combine_partial_kernel(const bf16* __restrict__ pair_out,
                                                              const int32_t* __restrict__ pidx,
                                                              const MoePlan* __restrict__ plan,
                                                              const int32_t* __restrict__ tok2u,
                                                              const bf16* __restrict__ remote,
                                                              const bf16* __restrict__ shared, bf16* __restrict__ out,
                                                              int K, int dim, HcPostArgs hp) {
  const int t = blockIdx.y, d = (blockIdx.x * 256 + threadIdx.x) * V;
  if (d >= dim) return;
  const int r0 = plan->remote0, u = tok2u[t];
  const bf16* rem = remote ? remote : pair_out + size_t(r0) * dim;
  float acc[8] = {};
  const auto add = [&](const bf16* p) {
    if constexpr (V == 8) {
      add_bf16x8(acc, p);
    } else {
      acc[0] += bf16_to_f32(*p);
    }
  };
  for (int j = 0; j < K; ++j) {
    const int p = pidx[size_t(t) * K + j];
    if (p < r0) add(pair_out + size_t(p) * dim + d);
  }
  if (u >= 0) add(rem + size_t(u) * dim + d);
  if (shared) add(shared + size_t(t) * dim + d);
  float o[8];
  if constexpr (V == 8) {
    const uint4 ov = pack_bf16x8(acc);
    *reinterpret_cast<uint4*>(out + size_t(t) * dim + d) = ov;
    const uint32_t w[4] = {ov.x, ov.y, ov.z, ov.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      o[2 * q] = __uint_as_float(w[q] << 16);
      o[2 * q + 1] = __uint_as_float(w[q] & 0xffff0000u);
    }
  } else {
    const bf16 ob = f32_to_bf16(acc[0]);
    out[size_t(t) * dim + d] = ob;
    o[0] = bf16_to_f32(ob);
  }
  if (!hp.x) return;
  const int hc = hp.hc;
  float r[4][8];
  for (int i = 0; i < hc; ++i) {
    const bf16* xp = hp.x + (size_t(t) * hc + i) * dim + d;
    if constexpr (V == 8) {
      const uint4 v = *reinterpret_cast<const uint4*>(xp);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        r[i][2 * q] = __uint_as_float(w[q] << 16);
        r[i][2 * q + 1] = __uint_as_float(w[q] & 0xffff0000u);
      }
    } else {
      r[i][0] = bf16_to_f32(*xp);
    }
  }
  for (int j = 0; j < hc; ++j) {
    const float pj = hp.post[size_t(t) * hc + j];
    float y[8];
#pragma unroll
    for (int c = 0; c < V; ++c) {
      float s = 0.0f;
      for (int i = 0; i < hc; ++i) s = fmaf(hp.comb[(size_t(t) * hc + i) * hc + j], r[i][c], s);
      y[c] = fmaf(pj, o[c], s);
    }
    bf16* xp = hp.x + (size_t(t) * hc + j) * dim + d;
    if constexpr (V == 8) {
      *reinterpret_cast<uint4*>(xp) = pack_bf16x8(y);
    } else {
      *xp = f32_to_bf16(y[0]);
    }
  }
}

__global__ __launch_bounds__(256) void gather_tokens16_kernel(const bf16* __restrict__ x, int dim,
                                                              const int32_t* __restrict__ u2t,
                                                              const MoePlan* __restrict__ plan, bf16* __restrict__ dst) {
  const int cols = dim / 8;
  const size_t n = size_t(plan->n_remote_tokens) * cols;
  for (size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x) {
    const size_t u = i / cols, c = i % cols;
    reinterpret_cast<uint4*>(dst + u * dim)[c] = reinterpret_cast<const uint4*>(x + size_t(u2t[u]) * dim)[c];
  }
  fence_system_once();
}

}  // namespace

// ---- entry points ---------------------------------------------------------------------------------------------------
void moe_count(const int32_t* sel, int T, int K, int32_t* count, int E, hipStream_t st, uint32_t* hist) {
  const int n = T * K;
  if (n <= 0) return;
  if (E > 0 && E <= 1024) moe_count_lds_kernel<<<cdiv(size_t(n), CNT_PER), CNT_NT, 0, st>>>(sel, n, E, count, hist);
  else moe_count_kernel<<<cdiv(size_t(n), 256), 256, 0, st>>>(sel, n, count, hist);
  UH_CHECK_LAUNCH();
}

void moe_plan(int32_t* count, const uint8_t* resident, int E, int P, MoePlan* plan, Exl3Tile* local_tiles,
              Exl3Tile* remote_tiles, int32_t* off, int32_t* fill, int max_tiles, hipStream_t st, int tile_rows) {
  if (E <= 0 || E > PLAN_NT) throw std::runtime_error("moe_plan: E must be in [1, 1024]");
  if (tile_rows <= 0 || tile_rows > kExl3TileRows) throw std::runtime_error("moe_plan: tile_rows in [1, 128]");
  moe_plan_kernel<<<1, PLAN_NT, 0, st>>>(count, resident, E, P, plan, local_tiles, remote_tiles, off, fill, max_tiles,
                                         tile_rows);
  UH_CHECK_LAUNCH();
}

void moe_scatter_e(const int32_t* sel, const float* wt, int T, int K, int E, const int32_t* off, int32_t* eidx,
                   float* ewt, int32_t* row_expert, int32_t* pidx, hipStream_t st) {
  if (T <= 0) return;
  if (K <= 0 || K > kMaxK || E <= 0) throw std::runtime_error("moe_scatter: K in [1, 8], E > 0");
  moe_scatter_kernel<<<unsigned(E), SC_NT, 0, st>>>(sel, wt, T, K, off, eidx, ewt, row_expert, pidx);
  UH_CHECK_LAUNCH();
}

// Without E: one block per possible expert id (< 1024, moe_plan's limit); a block whose id no token picked never
// reads off[] and writes nothing.
void moe_scatter(const int32_t* sel, const float* wt, int T, int K, const int32_t* off, int32_t*, int32_t* eidx,
                 float* ewt, int32_t* row_expert, int32_t* pidx, hipStream_t st) {
  moe_scatter_e(sel, wt, T, K, PLAN_NT, off, eidx, ewt, row_expert, pidx, st);
}

__global__ void zero_words_kernel(int32_t* p, size_t n) {
  for (size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x) p[i] = 0;
}

void launch_zero_words(int32_t* p, size_t n, hipStream_t st) {
  if (!n) return;
  zero_words_kernel<<<unsigned(std::min<size_t>(cdiv(n, 256), 1024)), 256, 0, st>>>(p, n);
  UH_CHECK_LAUNCH();
}

void moe_dispatch_small(const MoeSmallArgs& a, hipStream_t st) {
  if (a.T <= 0) return;
  if (a.T > kMoeSmallMaxTokens || a.K <= 0 || a.K > kMaxK) throw std::runtime_error("moe_dispatch_small: T <= 32, K <= 8");
  if (a.E <= 0 || a.E > 1024) throw std::runtime_error("moe_dispatch_small: E in [1, 1024]");
  if (a.P != a.T * a.K) throw std::runtime_error("moe_dispatch_small: P != T * K");
  if (a.tile_rows <= 0) throw std::runtime_error("moe_dispatch_small: tile_rows");
  if (a.resident && !a.rtl) throw std::runtime_error("moe_dispatch_small: a resident mask needs remote tiles");
  if (a.remote) {
    if (!a.resident) throw std::runtime_error("moe_dispatch_small: remote without a resident mask");
    if (!a.plan_dst || !a.tiles_dst || !a.w_dst || !a.e_dst) throw std::runtime_error("moe_dispatch_small: staging");
    if (a.qin && (!a.tok2u || !a.u2t || !a.p2u_dst)) throw std::runtime_error("moe_dispatch_small: remote tokens");
    if ((a.x_dst || a.q_dst) && !a.qin) throw std::runtime_error("moe_dispatch_small: x_dst / q_dst need qin");
    if ((a.x_dst || a.q_dst) && (!a.x || a.dim <= 0 || reinterpret_cast<uintptr_t>(a.x) % 16))
      throw std::runtime_error("moe_dispatch_small: x (16-byte aligned) and dim");
    if (a.x_dst && (a.dim % 8 || reinterpret_cast<uintptr_t>(a.x_dst) % 16))
      throw std::runtime_error("moe_dispatch_small: x_dst 16-byte aligned, dim % 8");
    if (a.q_dst && (a.dim % 128 || !a.qs_dst)) throw std::runtime_error("moe_dispatch_small: q_dst needs dim % 128");
  } else if (a.qin || a.x_dst || a.q_dst || a.req_flag || a.plan_dst) {
    throw std::runtime_error("moe_dispatch_small: remote-side outputs without remote");
  }
  if (!a.sel || !a.wt || !a.plan || !a.lt || !a.eidx || !a.ewt || !a.row_expert || !a.pidx)
    throw std::runtime_error("moe_dispatch_small: null output");
  moe_dispatch_small_kernel<<<1, SMALL_NT, 0, st>>>(a);
  UH_CHECK_LAUNCH();
}
void moe_dispatch_mid(const MoeSmallArgs& a, hipStream_t st) {
  static_assert(kMoeMidMaxPicks == SMALL_NT, "a thread per pick");
  if (a.T <= 0) return;
  if (a.K <= 0 || a.K > kMaxK || a.T * a.K > kMoeMidMaxPicks) throw std::runtime_error("moe_dispatch_mid: T * K <= 512, K <= 8");
  if (a.E <= 0 || a.E > 1024) throw std::runtime_error("moe_dispatch_mid: E in [1, 1024]");
  if (a.P != a.T * a.K) throw std::runtime_error("moe_dispatch_mid: P != T * K");
  if (a.tile_rows <= 0) throw std::runtime_error("moe_dispatch_mid: tile_rows");
  if (a.resident || a.remote || a.qin || a.x_dst || a.q_dst || a.req_flag || a.plan_dst)
    throw std::runtime_error("moe_dispatch_mid: local steps only");
  if (!a.sel || !a.wt || !a.plan || !a.lt || !a.eidx || !a.ewt || !a.row_expert || !a.pidx)
    throw std::runtime_error("moe_dispatch_mid: null output");
  moe_dispatch_small_kernel<<<1, SMALL_NT, 0, st>>>(a);
  UH_CHECK_LAUNCH();
}

namespace {
unsigned stride_grid(size_t units) { return unsigned(std::max<size_t>(1, std::min<size_t>(cdiv(units, 256), 1024))); }
bool a16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }
}  // namespace

void moe_trace(const int32_t* sel, int n, uint8_t* dst, hipStream_t st) {
  if (n <= 0) return;
  if (!sel || !dst) throw std::runtime_error("moe_trace: null operand");
  moe_trace_kernel<<<unsigned(cdiv(size_t(n), 256)), 256, 0, st>>>(sel, n, dst);
  UH_CHECK_LAUNCH();
}
void stage_remote(const MoePlan* plan, const Exl3Tile* rtiles, const float* ewt, const int32_t* row_expert,
                  MoePlan* plan_dst, Exl3Tile* tiles_dst, float* w_dst, int32_t* e_dst, int max_rows, hipStream_t st) {
  if (!plan || !rtiles || !ewt || !row_expert || !plan_dst || !tiles_dst || !w_dst || !e_dst)
    throw std::runtime_error("stage_remote: null operand");
  stage_remote_kernel<<<stride_grid(std::max(max_rows, 1)), 256, 0, st>>>(plan, rtiles, ewt, row_expert, plan_dst,
                                                                          tiles_dst, w_dst, e_dst, true);
  UH_CHECK_LAUNCH();
}
void copy_remote_meta(const float* ewt, const int32_t* row_expert, float* w_dst, int32_t* e_dst, const MoePlan* plan,
                      int max_rows, hipStream_t st) {
  if (!plan || !ewt || !row_expert || !w_dst || !e_dst) throw std::runtime_error("copy_remote_meta: null operand");
  stage_remote_kernel<<<stride_grid(std::max(max_rows, 1)), 256, 0, st>>>(plan, nullptr, ewt, row_expert, nullptr,
                                                                          nullptr, w_dst, e_dst, false);
  UH_CHECK_LAUNCH();
}
void copy_remote_rows(const uint16_t* src, uint16_t* dst, const MoePlan* plan, int dim, int max_rows, hipStream_t st) {
  if (dim <= 0 || dim % 8 || !a16(src) || !a16(dst) || !plan)
    throw std::runtime_error("copy_remote_rows: dim % 8, 16-byte aligned rows");
  copy_rows16_kernel<<<stride_grid(size_t(std::max(max_rows, 1)) * (dim / 8)), 256, 0, st>>>(
      reinterpret_cast<const uint4*>(src), reinterpret_cast<uint4*>(dst), plan, dim / 8, 0);
  UH_CHECK_LAUNCH();
}
void copy_remote_partial(const uint16_t* src, uint16_t* dst, const MoePlan* plan, int dim, int max_tokens,
                         hipStream_t st) {
  if (dim <= 0 || dim % 8 || !a16(src) || !a16(dst) || !plan)
    throw std::runtime_error("copy_remote_partial: dim % 8, 16-byte aligned rows");
  copy_rows16_kernel<<<stride_grid(size_t(std::max(max_tokens, 1)) * (dim / 8)), 256, 0, st>>>(
      reinterpret_cast<const uint4*>(src), reinterpret_cast<uint4*>(dst), plan, dim / 8, 1);
  UH_CHECK_LAUNCH();
}
void copy_remote_tokens(const uint16_t* x, int dim, const int32_t* u2t, const MoePlan* plan, uint16_t* dst,
                        int max_tokens, hipStream_t st) {
  if (max_tokens <= 0) return;
  if (dim <= 0 || dim % 8 || !a16(x) || !a16(dst) || !u2t || !plan)
    throw std::runtime_error("copy_remote_tokens: dim % 8, 16-byte aligned rows");
  gather_tokens16_kernel<<<stride_grid(size_t(max_tokens) * (dim / 8)), 256, 0, st>>>(x, dim, u2t, plan, dst);
  UH_CHECK_LAUNCH();
}
void remote_tokens(const int32_t* pidx, const int32_t* eidx, int T, int K, MoePlan* plan, int32_t* tok2u,
                   int32_t* u2t, int32_t* p2u_dst, int32_t* u2p_dst, hipStream_t st) {
  if (T < 0 || K <= 0) throw std::runtime_error("remote_tokens: T >= 0, K >= 1");
  if (!pidx || !eidx || !plan || !tok2u || !u2t || !p2u_dst) throw std::runtime_error("remote_tokens: null operand");
  remote_tokens_kernel<<<1, RT_NT, 0, st>>>(pidx, eidx, T, K, plan, tok2u, u2t, p2u_dst, u2p_dst);
  UH_CHECK_LAUNCH();
}
void remote_combine(const uint16_t* pair_out, const int32_t* u2p, const MoePlan* plan, uint16_t* dst, int K, int dim,
                    int max_tokens, hipStream_t st) {
  launch_remote_combine(pair_out, dim, u2p, plan, dst, K, dim, max_tokens, st);
}
void launch_remote_combine(const uint16_t* pair_out, int ld, const int32_t* u2p, const MoePlan* plan, uint16_t* dst,
                           int K, int dim, int max_tokens, hipStream_t st) {
  if (max_tokens <= 0) return;
  if (dim <= 0 || dim % 8 || ld < dim || ld % 8 || !a16(pair_out) || !a16(dst))
    throw std::runtime_error("remote_combine: dim % 8, ld % 8, 16-byte aligned rows");
  if (!u2p || !plan || K <= 0) throw std::runtime_error("remote_combine: null operand");
  remote_combine_kernel<<<dim3(unsigned(cdiv(size_t(dim / 8), 256)), unsigned(std::min(max_tokens, 256))), 256, 0,
                          st>>>(
      pair_out, u2p, plan, dst, K, dim, ld);
  UH_CHECK_LAUNCH();
}
namespace {
void launch_combine_partial(const uint16_t* pair_out, const int32_t* pidx, const MoePlan* plan, const int32_t* tok2u,
                            const uint16_t* remote, const uint16_t* shared, uint16_t* out, int T, int K, int dim,
                            const HcPostArgs& hp, hipStream_t st) {
  if (T <= 0) return;
  if (dim <= 0 || K <= 0 || !pair_out || !pidx || !plan || !tok2u || !out)
    throw std::runtime_error("moe_combine_partial: null operand or shape");
  if (hp.x && (!hp.post || !hp.comb || hp.hc < 1 || hp.hc > 4))
    throw std::runtime_error("moe_combine_partial: mHC post-mix needs post, comb and 1 <= hc <= 4");
  const bool v8 = dim % 8 == 0 && a16(pair_out) && a16(out) && (!remote || a16(remote)) && (!shared || a16(shared)) &&
                  (!hp.x || a16(hp.x));
  if (v8)
    combine_partial_kernel<8><<<dim3(unsigned(cdiv(size_t(dim / 8), 256)), unsigned(T)), 256, 0, st>>>(
        pair_out, pidx, plan, tok2u, remote, shared, out, K, dim, hp);
  else
    combine_partial_kernel<1><<<dim3(unsigned(cdiv(size_t(dim), 256)), unsigned(T)), 256, 0, st>>>(
        pair_out, pidx, plan, tok2u, remote, shared, out, K, dim, hp);
  UH_CHECK_LAUNCH();
}
}  // namespace
void moe_combine_partial(const uint16_t* pair_out, const int32_t* pidx, const MoePlan* plan, const int32_t* tok2u,
                         const uint16_t* shared, uint16_t* out, int T, int K, int dim, hipStream_t st) {
  launch_combine_partial(pair_out, pidx, plan, tok2u, nullptr, shared, out, T, K, dim, HcPostArgs{}, st);
}
void moe_combine_partial_link(const uint16_t* pair_out, const int32_t* pidx, const MoePlan* plan, const int32_t* tok2u,
                              const uint16_t* remote, const uint16_t* shared, uint16_t* out, int T, int K, int dim,
                              hipStream_t st, const HcPostArgs& hp) {
  if (!remote) throw std::runtime_error("moe_combine_partial_link: null remote rows");
  launch_combine_partial(pair_out, pidx, plan, tok2u, remote, shared, out, T, K, dim, hp, st);
}

void route(const float* logits, const float* bias, const int32_t* tid2eid, const int32_t* ids, int32_t* sel,
           float* weights, int T, int E, int K, float route_scale, hipStream_t st, const float* bias_vl, int vocab) {
  if (T <= 0) return;
  if (K <= 0 || K > kMaxK || K > E) throw std::runtime_error("route: K in [1, 8], K <= E");
  route_thread_kernel<<<cdiv(size_t(T), 64), 64, 0, st>>>(logits, bias, tid2eid, ids, sel, weights, T, E, K,
                                                           route_scale, bias_vl, vocab);
  UH_CHECK_LAUNCH();
}
void route_fast(const float* logits, const float* bias, const int32_t* tid2eid, const int32_t* ids, int32_t* sel,
                float* weights, int T, int E, int K, float route_scale, hipStream_t st, const float* bias_vl,
                int vocab) {
  if (T <= 0) return;
  if (E > 1024 || K <= 0 || K > kMaxK || K > E) throw std::runtime_error("route_fast: E <= 1024, K in [1, 8]");
  route_wave_kernel<0><<<cdiv(size_t(T), 4), 256, 0, st>>>(logits, bias, tid2eid, ids, sel, weights, T, E, K,
                                                            route_scale, bias_vl, vocab);
  UH_CHECK_LAUNCH();
}
void route_glm(const float* logits, const float* bias, int32_t* sel, float* weights, int T, int E, int K,
               float route_scale, hipStream_t st) {
  if (T <= 0) return;
  if (E > 1024 || K <= 0 || K > kMaxK || K > E) throw std::runtime_error("route_glm: E <= 1024, K in [1, 8]");
  route_wave_kernel<1><<<cdiv(size_t(T), 4), 256, 0, st>>>(logits, bias, nullptr, nullptr, sel, weights, T, E, K,
                                                            route_scale, nullptr, 0);
  UH_CHECK_LAUNCH();
}
void route_softmax(const float* logits, int32_t* sel, float* weights, int T, int E, int K, hipStream_t st) {
  if (T <= 0) return;
  if (E > 1024 || K <= 0 || K > kMaxK || K > E) throw std::runtime_error("route_softmax: E <= 1024, K in [1, 8]");
  route_wave_kernel<2><<<cdiv(size_t(T), 4), 256, 0, st>>>(logits, nullptr, nullptr, nullptr, sel, weights, T, E, K,
                                                            1.0f, nullptr, 0);
  UH_CHECK_LAUNCH();
}

void swiglu(const bf16* gate, const bf16* up, const float* w, bf16* h, int rows, int dim, float limit,
            hipStream_t st) {
  if (rows <= 0) return;
  swiglu_kernel<<<cdiv(size_t(rows) * dim, 256), 256, 0, st>>>(gate, up, w, h, rows, dim, limit);
  UH_CHECK_LAUNCH();
}
void gather_rows(const bf16* src, const int32_t* rows_idx, bf16* dst, int n, int dim, hipStream_t st) {
  if (n <= 0) return;
  gather_rows_kernel<<<cdiv(size_t(n) * dim, 256), 256, 0, st>>>(src, rows_idx, dst, n, dim);
  UH_CHECK_LAUNCH();
}
void scatter_add(const bf16* src, const int32_t* rows_idx, float* y, int n, int dim, hipStream_t st) {
  if (n <= 0) return;
  scatter_add_kernel<<<cdiv(size_t(dim), 256), 256, 0, st>>>(src, rows_idx, y, n, dim);
  UH_CHECK_LAUNCH();
}
void moe_combine(const bf16* pair_out, const int32_t* pidx, const bf16* shared, bf16* out, int T, int K, int dim,
                 hipStream_t st) {
  if (T <= 0) return;
  if (dim % 8) throw std::runtime_error("moe_combine: dim % 8");
  moe_combine_kernel<<<dim3(cdiv(size_t(dim), 2048), unsigned(T)), 256, 0, st>>>(pair_out, pidx, shared, out, K, dim);
  UH_CHECK_LAUNCH();
}

}  // namespace unholy::kernels
