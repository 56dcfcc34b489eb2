// MXFP4 routed-expert kernels for gfx950: layout repack, activation transforms, the grouped GEMV for decode /
// verify tiles and its SwiGLU epilogue, and the MFMA decode self-check. The prefill grouped GEMM is in
// mx_gemm.hip. Entry points and layouts: include/unholy/kernels/mx_moe.hpp.
#include <algorithm>
#include <cstdlib>
#include <string>

#include "common.hpp"
#include "numerics.hpp"
#include "unholy/kernels/mx_moe.hpp"
#include "mx_internal.hpp"

namespace unholy::kernels {

using namespace uh;

namespace {

// One thread per (row n, 16-byte piece p of the row's K/2 code bytes), which is also one scale byte (K/32 of
// each per row): the piece goes to chunk (p/2) * (N/16) + n/16 at (n % 16) * 32 + (p % 2) * 16, the scale
// byte b = p to chunk (b/2) * (N/16) + n/16 at (n % 16) * 2 + b % 2 (ref mx_moe.hip:82-96, expert_pack.cpp:146-166).
__global__ __launch_bounds__(256) void mx_repack_kernel(const uint8_t* __restrict__ w, const uint8_t* __restrict__ s,
                                                        uint8_t* __restrict__ tw, uint8_t* __restrict__ ts, int N,
                                                        int K) {
  const size_t gid = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  const int per_row = K / 32;
  if (gid >= size_t(N) * per_row) return;
  const int n = int(gid / per_row), p = int(gid % per_row);
  const size_t chunk = size_t(p / 2) * (N / 16) + n / 16;
  *reinterpret_cast<uint4*>(tw + chunk * 512 + (n % 16) * 32 + (p % 2) * 16) =
      *reinterpret_cast<const uint4*>(w + gid * 16);
  ts[chunk * 32 + (n % 16) * 2 + p % 2] = s[gid];
}

// Activation transforms on a wave per (row, 128-value segment), two values per lane, items striding over the
// grid. kMode 0: x rows -> fake-quantized bf16 (mx_xform_in); 1: x rows -> e4m3 codes + e8m0 scale
// (mx_xform_in_fp8); 2: g/u rows -> bf16 SwiGLU -> fake-quantized bf16 and/or codes (mx_swiglu). Rows whose
// expert's scale-table entry is null are skipped (ref mx_moe.hip:132-179).
template <int kMode>
__global__ __launch_bounds__(256) void mx_transform_kernel(const bf16* __restrict__ x, int ldx,
                                                           const int32_t* __restrict__ x_rows,
                                                           const bf16* __restrict__ u, const float* __restrict__ w,
                                                           float limit, const int32_t* __restrict__ row_expert,
                                                           const uint8_t* const* __restrict__ s_tab,
                                                           bf16* __restrict__ out, uint8_t* __restrict__ q,
                                                           uint8_t* __restrict__ qs, int K, int P) {
  const int lane = threadIdx.x & 63, segs = K / 128;
  const size_t n = size_t(P) * segs;
  for (size_t it = size_t(blockIdx.x) * 4 + (threadIdx.x >> 6); it < n; it += size_t(gridDim.x) * 4) {
    const int r = int(it / segs), seg = int(it % segs), k0 = seg * 128 + 2 * lane;
    if (s_tab && !s_tab[row_expert[r]]) continue;  // uniform per wave
    float v[2];
    if constexpr (kMode == 2) {
      const uint32_t graw = *reinterpret_cast<const uint32_t*>(x + size_t(r) * ldx + k0);
      const uint32_t uraw = *reinterpret_cast<const uint32_t*>(u + size_t(r) * ldx + k0);
#pragma unroll
      for (int i = 0; i < 2; ++i)
        v[i] = round_bf16(swiglu_value(bf16_to_f32(uint16_t(graw >> (16 * i))), bf16_to_f32(uint16_t(uraw >> (16 * i))),
                                       w ? w[r] : 0.0f, w != nullptr, limit));
    } else {
      const size_t src = x_rows ? size_t(x_rows[r]) : size_t(r);
      const uint32_t raw = *reinterpret_cast<const uint32_t*>(x + src * ldx + k0);
      v[0] = bf16_to_f32(uint16_t(raw));
      v[1] = bf16_to_f32(uint16_t(raw >> 16));
    }
    const Fp8Block b = fp8_block_scale(wave_max(fmaxf(fabsf(v[0]), fabsf(v[1]))));
    const uint8_t c0 = fp8_code(v[0], b), c1 = fp8_code(v[1], b);
    if (out)
      *reinterpret_cast<uint32_t*>(out + size_t(r) * K + k0) =
          uint32_t(f32_to_bf16(e4m3_to_f32(c0) * b.sc)) | uint32_t(f32_to_bf16(e4m3_to_f32(c1) * b.sc)) << 16;
    if (q) {
      *reinterpret_cast<uint16_t*>(q + size_t(r) * K + k0) = uint16_t(c0 | uint32_t(c1) << 8);
      if (lane == 0) qs[size_t(r) * segs + seg] = b.se;
    }
  }
}

// The same transforms with 8 values per thread: 16 consecutive threads cover one 128-value segment (16-byte loads,
// 8- or 16-byte stores), its amax a DPP row max. The item loop has a uniform bound so that every 16-lane group is
// whole; threads past the end work on the last item and store nothing. Needs 16-byte aligned rows (ldx % 8 == 0).
template <int kMode>
__global__ __launch_bounds__(256) void mx_transform8_kernel(const bf16* __restrict__ x, int ldx,
                                                            const int32_t* __restrict__ x_rows,
                                                            const bf16* __restrict__ u, int ldu,
                                                            const float* __restrict__ w,
                                                            float limit, const int32_t* __restrict__ row_expert,
                                                            const uint8_t* const* __restrict__ s_tab,
                                                            bf16* __restrict__ out, uint8_t* __restrict__ q,
                                                            uint8_t* __restrict__ qs, int K, int P) {
  const int segs = K / 128;
  const size_t per_row = size_t(segs) * 16, items = size_t(P) * per_row;
  for (size_t base = size_t(blockIdx.x) * 256; base < items; base += size_t(gridDim.x) * 256) {
    const size_t it = min(base + threadIdx.x, items - 1);
    const int r = int(it / per_row), rem = int(it % per_row), seg = rem >> 4, k0 = seg * 128 + (rem & 15) * 8;
    float v[8];
    if constexpr (kMode == 2) {
      const uint4 graw = *reinterpret_cast<const uint4*>(x + size_t(r) * ldx + k0);
      const uint4 uraw = *reinterpret_cast<const uint4*>(u + size_t(r) * ldu + k0);
      const uint32_t gw[4] = {graw.x, graw.y, graw.z, graw.w}, uw[4] = {uraw.x, uraw.y, uraw.z, uraw.w};
      const float wr = w ? w[r] : 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        v[i] = round_bf16(swiglu_value(bf16_to_f32(uint16_t(gw[i / 2] >> (16 * (i % 2)))),
                                       bf16_to_f32(uint16_t(uw[i / 2] >> (16 * (i % 2)))), wr, w != nullptr, limit));
    } else {
      const size_t src = x_rows ? size_t(x_rows[r]) : size_t(r);
      const uint4 raw = *reinterpret_cast<const uint4*>(x + src * ldx + k0);
      const uint32_t rw[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float(rw[i] << 16);
        v[2 * i + 1] = __uint_as_float(rw[i] & 0xffff0000u);
      }
    }
    float am = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) am = fmaxf(am, fabsf(v[i]));
    const Fp8Block b = fp8_block_scale(row16_max(am));
    if (base + threadIdx.x >= items || (s_tab && !s_tab[row_expert[r]])) continue;
    uint32_t c[2];
    fp8_codes8(v, b, c[0], c[1]);
    if (out)  // the fake-quantized values: the codes decoded back (exact)
      *reinterpret_cast<uint4*>(out + size_t(r) * K + k0) = __builtin_bit_cast(uint4, fp8x8_to_bf16(c[0], c[1], b.sc));
    if (q) {
      *reinterpret_cast<uint2*>(q + size_t(r) * K + k0) = make_uint2(c[0], c[1]);
      if ((rem & 15) == 0) qs[size_t(r) * segs + seg] = b.se;
    }
  }
}

unsigned transform_blocks(int P, int K) { return unsigned(std::min<size_t>((size_t(P) * (K / 128) + 3) / 4, 16384)); }

// ---- grouped GEMV ----------------------------------------------------------------------------------------------------
// A workgroup = 8 waves x one 16-output tile each = 128 outputs of one tile (one expert's run of <= 16 pair rows), for
// one or two projections (w1 and w3 of the same rows). The tile's rows are staged once into LDS as e4m3 codes + e8m0
// scales (copied from the fp8 form, or recovered exactly from fake-quantized bf16 rows); then every wave streams its
// weight columns straight from HBM into registers, GV_PF 128-input steps ahead of use: per step, lane l takes the
// 16 code bytes of column l % 16, inputs 32 (l / 16) .. + 31 (chunk 2s + (l/16)/2 at (l % 16) * 32 + ((l/16) % 2)
// * 16: each half-wave reads one contiguous 512-byte chunk of the tile-major layout) and that 32-block's scale
// byte, dequantizes them exactly to bf16 with the scaled conversion instructions and issues four bf16 MFMAs against
// the matching activation inputs. The MFMA accumulates in fp32 with exact products; no cross-lane reductions.
// GV_PF: weight steps in flight per wave (8 measured slower: the larger ring costs occupancy).
constexpr int GV_WAVES = 8, GV_PAD = 16, GV_MAXROWS = 16, GV_PF = 4;
// The live tile count of a launch without a device-side count.
__device__ const int g_no_tile_limit = 0x7fffffff;

// AM: activation source -- 0: e4m3 codes + e8m0 scales (aq, as); 1: fake-quantized bf16 rows (xa), codes recovered
// exactly; 2: raw bf16 token rows x[x_rows[r]] quantized here with the reference's act_quant (mx_xform_in_fp8 fused).
// GM: epilogue -- 0: plain outputs; 1: SwiGLU + fp8 requantization of each row's 128-output block (W = 8 waves
// cover the block); 2: SwiGLU to raw bf16 rows h (no requantization: the consumer quantizes them while staging).
// W: waves per workgroup (16 outputs each).
// KSPLIT (small launches, plain outputs): the workgroup is one 16-column tile whose W waves take K / W steps each, so
// every wave's weight loads are in flight at once; the partial sums are added in LDS in wave order.
// ABF: the staged rows are held as their bf16 values (the codes times their e8m0 scale, exact) instead of codes +
// scales, so each step reads its activation operands without converting them; rows past the tile read a zero row.
// Chosen when (rows_cap + 1) rows of bf16 fit the LDS.
template <int NP, int GM, int AM, int W, bool KSPLIT = false, bool ABF = false>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(2))) void mx_gemv_kernel(MxGemvArgs a) {
  static_assert(!KSPLIT || GM == 0, "the K split has a plain epilogue");
  static_assert(!(KSPLIT && ABF), "the K split stages codes");
  constexpr int NT = 64 * W;
  extern __shared__ __align__(16) uint8_t smem[];
  // The tile and the live tile count are loaded together (the tile slot is in bounds: the grid has one row per
  // slot), then the expert's table entries, then the weights: three dependent loads before the first weight byte
  // instead of five.
  const Exl3Tile tile = a.tiles[blockIdx.y];
  const int live = *(a.ntiles_dev ? a.ntiles_dev : &g_no_tile_limit);
  // The arguments the weight stream's first addresses need, read with the tile rather than one after another
  // behind the table entries.
  asm volatile("" ::"s"(a.K), "s"(a.N), "s"(a.ldo), "s"(a.rows_cap), "s"(a.split), "s"(a.w_tab[0]), "s"(a.s_tab[0]),
               "s"(a.w_tab[1]), "s"(a.s_tab[1]), "s"(a.aq), "s"(a.as), "s"(a.xa), "s"(a.out[0]), "s"(a.out32));
  if (int(blockIdx.y) >= live || tile.rows <= 0 || tile.expert < 0) return;  // all three fields in one load
  const uint8_t* wp[NP];
  const uint8_t* sp[NP];
  wp[0] = a.w_tab[0][tile.expert];
  sp[0] = a.s_tab[0][tile.expert];
  if constexpr (NP == 2) {
    if (a.split) {  // the same matrix from column tile `split` on
      wp[1] = wp[0] ? wp[0] + size_t(a.split) * 512 : nullptr;
      sp[1] = sp[0] ? sp[0] + size_t(a.split) * 32 : nullptr;
    } else {
      wp[1] = a.w_tab[1][tile.expert];
      sp[1] = a.s_tab[1][tile.expert];
    }
  }
#pragma unroll
  for (int p = 0; p < NP; ++p)
    if (!wp[p] || !sp[p]) return;
  const int K = a.K, N = a.N, KS = K / 128, ldA = K + GV_PAD, ntn = N / 16;
  uint8_t* sA = smem;
  uint8_t* sS = smem + size_t(a.rows_cap) * ldA;
  uint16_t* const sAb = reinterpret_cast<uint16_t*>(smem);  // ABF: [rows_cap + 1][ldAb] bf16, the last row zero
  const int ldAb = K + 8;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, nl = lane & 15, g = lane >> 4;
  if constexpr (ABF)
    for (int i = tid * 8; i < ldAb; i += NT * 8)
      *reinterpret_cast<uint4*>(sAb + size_t(a.rows_cap) * ldAb + i) = uint4{0u, 0u, 0u, 0u};
  const int nt = KSPLIT ? int(blockIdx.x) : int(blockIdx.x) * W + wave;
  const bool active = nt < (a.split ? a.split : ntn);  // uniform per wave
  const int sb = KSPLIT ? wave * (KS / W) : 0, se = KSPLIT ? sb + KS / W : KS;  // this wave's K steps
  const int boff = nl * 32 + (g & 1) * 16;
  for (int rg = 0; rg < tile.rows; rg += a.rows_cap) {
    const int M = min(a.rows_cap, tile.rows - rg);
    const size_t row0 = size_t(tile.row0) + rg;
    // Prefetch the first GV_PF steps of weights before staging the activations (independent of them).
    v4i bq[GV_PF][NP];
    // 32-bit offsets from the (uniform) matrix base: loads take the scalar-base + vector-offset form.
    const uint32_t cofs = uint32_t(((g >> 1) * ntn + nt) * 512 + boff);
    const uint32_t cstep = uint32_t(2 * ntn * 512);
    const auto load_step = [&](int s, int slot) {
#pragma unroll
      for (int p = 0; p < NP; ++p)  // streamed once per launch: nontemporal loads (~12% more read bandwidth)
        bq[slot][p] = __builtin_nontemporal_load(reinterpret_cast<gptr<v4i>>(as_global(wp[p]) + (cofs + uint32_t(s) * cstep)));
    };
    // Weight scales per 4 steps (8 slabs of 64 inputs): lane l loads dword l % 8 of slab l / 8's 32-byte scale chunk
    // of the wave's 16 columns -- one load per projection per 4 steps instead of a byte per step. A step's byte is
    // then taken from the owning lane with ds_bpermute (the lane crossbar, no memory access). These loads go
    // through the caches: the workgroup's waves read neighbouring 32-byte pieces of one 128-byte line (nontemporal
    // 32-byte reads cost ~4% of the launch's time in a load-only measurement of this pattern).
    constexpr int SW = GV_PF / 4;
    static_assert(GV_PF % 4 == 0, "a scale dword per lane covers 4 steps");
    uint32_t sq_cur[SW][NP], sq_nxt[SW][NP];
    const auto load_scales = [&](int s0, uint32_t (&dst)[SW][NP]) {
#pragma unroll
      for (int j = 0; j < SW; ++j) {
        const uint32_t slab = uint32_t(min(2 * (s0 + 4 * j) + (lane >> 3), 2 * KS - 1));
        const uint32_t so = (slab * uint32_t(ntn) + uint32_t(nt)) * 32u + uint32_t(lane & 7) * 4u;
#pragma unroll
        for (int p = 0; p < NP; ++p) dst[j][p] = *reinterpret_cast<gptr<uint32_t>>(as_global(sp[p]) + so);
      }
    };
    if (active) {
      load_scales(sb, sq_cur);
#pragma unroll
      for (int i = 0; i < GV_PF; ++i) load_step(min(sb + i, se - 1), i);  // fewer than GV_PF steps: re-read the last
    }
    __syncthreads();
    if constexpr (AM == 1 && ABF) {
      // bf16 rows held as they are: for fake-quantized rows (mx_xform_in's) these are exactly the values the codes
      // and scales recovered below would give back, and other bf16 rows are used as given.
      const int total = M * (K / 8);
      for (int i = tid; i < total; i += NT) {
        const int m = i / (K / 8), c = (i % (K / 8)) * 8;
        *reinterpret_cast<uint4*>(sAb + m * ldAb + c) = *reinterpret_cast<const uint4*>(a.xa + (row0 + m) * size_t(K) + c);
      }
    } else if constexpr (AM != 0) {
      // 8 values per thread; 16 consecutive threads hold one 128-block (K / 8 is a multiple of 16).
      const int total = M * (K / 8);
      for (int base = 0; base < total; base += NT) {
        const int i = base + tid, m = i / (K / 8), c = (i % (K / 8)) * 8;
        const bool valid = i < total;
        float v[8];
        float am = 0.0f;
        if (valid) {
          const uint16_t* src = AM == 1 ? a.xa + (row0 + m) * size_t(K)
                                        : a.xa + size_t(a.x_rows ? a.x_rows[row0 + m] : int(row0 + m)) * a.ldx;
          const uint4 raw = *reinterpret_cast<const uint4*>(src + c);
          const uint32_t r4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            v[2 * t] = __uint_as_float(r4[t] << 16);
            v[2 * t + 1] = __uint_as_float(r4[t] & 0xffff0000u);
          }
#pragma unroll
          for (int t = 0; t < 8; ++t) am = fmaxf(am, fabsf(v[t]));
        }
        am = group_max<16>(am);
        if (valid) {
          uint8_t se;
          uint32_t lo, hi;
          if constexpr (AM == 1) {
            se = uint8_t(min(max(int(exact_fp8_scale(am)), 1), 254));
            const float inv = e8m0_to_f32(uint8_t(254 - se));  // 2^(127 - se), exact
            lo = e4m3x4(v[0] * inv, v[1] * inv, v[2] * inv, v[3] * inv);  // exact values: |v * inv| <= 448
            hi = e4m3x4(v[4] * inv, v[5] * inv, v[6] * inv, v[7] * inv);
          } else {
            const Fp8Block blk = fp8_block_scale(am);
            se = blk.se;
            fp8_codes8(v, blk, lo, hi);
          }
          if constexpr (ABF) {
            *reinterpret_cast<bf16x8*>(sAb + m * ldAb + c) = fp8x8_to_bf16(lo, hi, e8m0_to_f32(se));
          } else {
            *reinterpret_cast<uint2*>(sA + m * ldA + c) = make_uint2(lo, hi);
            if ((c & 127) == 0) sS[m * KS + c / 128] = se;
          }
        }
      }
    } else {
      const int total = M * (K / 16);
      for (int i = tid; i < total; i += NT) {
        const int m = i / (K / 16), c = (i % (K / 16)) * 16;
        const uint4 q = *reinterpret_cast<const uint4*>(a.aq + (row0 + m) * K + c);
        if constexpr (ABF) {
          const float sc = e8m0_to_f32(a.as[(row0 + m) * KS + c / 128]);
          *reinterpret_cast<bf16x8*>(sAb + m * ldAb + c) = fp8x8_to_bf16(q.x, q.y, sc);
          *reinterpret_cast<bf16x8*>(sAb + m * ldAb + c + 8) = fp8x8_to_bf16(q.z, q.w, sc);
        } else {
          *reinterpret_cast<uint4*>(sA + m * ldA + c) = q;
        }
      }
      if constexpr (!ABF)
        for (int i = tid; i < M * KS; i += NT) sS[i] = a.as[row0 * KS + i];
    }
    __syncthreads();

    v4f acc[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) acc[p] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    const bool arow = nl < M;
    const uint8_t* ap = sA + nl * ldA + g * 8;
    const uint8_t* asp = sS + nl * KS;
    // One step (128 inputs = four 32-blocks): MFMA t sums block t of the step, so that every output accumulates
    // acc + (block sum) x (scales) block after block in input order, the reference's order (ref_gemm.hip:54-63: the
    // 32 products are exact, their sum is exact in fp32 and the MFMA adds it with one rounding). Lane (nl, g)
    // supplies inputs 8g .. 8g + 7 of block t on both sides. The weights arrive as block g of the step in lane group
    // g (16 bytes); a 4 x 4 transpose of dwords across the lane groups (two permlane32 and two permlane16 swaps)
    // hands each group its dword of every block.
    const uint16_t* apb = sAb + size_t(arow ? nl : a.rows_cap) * ldAb + g * 8;
    const auto step = [&](int s, int i) {
      bf16x8 af[4];
      if constexpr (ABF) {
#pragma unroll
        for (int t = 0; t < 4; ++t) af[t] = *reinterpret_cast<const bf16x8*>(apb + s * 128 + 32 * t);
      } else if (arow) {
        const float sc = e8m0_to_f32(asp[s]);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const uint2 v = *reinterpret_cast<const uint2*>(ap + s * 128 + 32 * t);
          af[t] = fp8x8_to_bf16(v.x, v.y, sc);
        }
      } else {
#pragma unroll
        for (int t = 0; t < 4; ++t) af[t] = bf16x8{};
      }
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        // the scale bytes of column nl in slabs 2 (i % 4) and 2 (i % 4) + 1 (dword nl / 2 of each, bytes
        // 2 (nl % 2) + h): blocks t = 2 slab' + h of the step
        uint32_t sw[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int src = ((2 * (i % 4) + j) * 8 + (nl >> 1)) * 4;
          sw[j] = uint32_t(__builtin_amdgcn_ds_bpermute(src, int(sq_cur[i / 4][p]))) >> (16 * (nl & 1));
        }
        const auto r02 = __builtin_amdgcn_permlane32_swap(uint32_t(bq[i][p][0]), uint32_t(bq[i][p][2]), false, false);
        const auto r13 = __builtin_amdgcn_permlane32_swap(uint32_t(bq[i][p][1]), uint32_t(bq[i][p][3]), false, false);
        const auto r01 = __builtin_amdgcn_permlane16_swap(r02[0], r13[0], false, false);
        const auto r23 = __builtin_amdgcn_permlane16_swap(r02[1], r13[1], false, false);
        const uint32_t wd[4] = {r01[0], r01[1], r23[0], r23[1]};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float sc = __uint_as_float(((sw[t >> 1] >> (8 * (t & 1))) & 0xffu) << 23);
          acc[p] = mfma_bf16(af[t], fp4x8_to_bf16(wd[t], sc), acc[p]);
        }
      }
    };
    if (active) {
      int s0 = sb;
      // Every round but the last loads the next round's weights. The loads are unconditional (a conditional load
      // would leave the compiler unsure how many are outstanding, and it would then wait for all of them each
      // round); with K % 512 == 0 none of them is past the end (otherwise they re-read the last step).
      for (; s0 + GV_PF < se; s0 += GV_PF) {
#pragma unroll
        for (int i = 0; i < GV_PF; ++i) {
          if (s0 + i < se) step(s0 + i, i);
          load_step(min(s0 + i + GV_PF, se - 1), i);
          if (i == 0) load_scales(s0 + GV_PF, sq_nxt);
          // Keep each step's conversions and MFMAs together: interleaving the unrolled steps would only raise
          // register pressure (the loads of later steps are already in flight).
          __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int j = 0; j < SW; ++j)
#pragma unroll
          for (int p = 0; p < NP; ++p) sq_cur[j][p] = sq_nxt[j][p];
      }
#pragma unroll
      for (int i = 0; i < GV_PF; ++i) {  // the last round: nothing left to load
        if (s0 + i < se) step(s0 + i, i);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if constexpr (KSPLIT) {  // the W partial sums of the tile, added in wave order, into wave 0
      __syncthreads();      // every wave is past its reads of the staged rows
      v4f* red = reinterpret_cast<v4f*>(smem);
#pragma unroll
      for (int p = 0; p < NP; ++p) red[(wave * NP + p) * 64 + lane] = acc[p];
      __syncthreads();
      if (wave == 0)
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          v4f t = red[p * 64 + lane];
#pragma unroll
          for (int w = 1; w < W; ++w) t += red[(w * NP + p) * 64 + lane];
          acc[p] = t;
        }
    }

    if constexpr (GM == 0) {
      if (active && (!KSPLIT || wave == 0))
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = 4 * g + i;
            if (r >= M) continue;
            const size_t o = (row0 + r) * a.ldo + nt * 16 + nl;
            if (p == 0 && a.out32) a.out32[o] = acc[p][i];
            else a.out[p][o] = f32_to_bf16(acc[p][i]);
          }
    } else if constexpr (GM == 2) {
      if (active)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 4 * g + i;
          if (r >= M) continue;
          const size_t row = row0 + r, col = size_t(nt) * 16 + nl;
          if (a.gs_tab && !a.gs_tab[a.grow_expert[row]]) continue;
          const float gv = round_bf16(acc[0][i]), uv = round_bf16(acc[NP - 1][i]);
          if (a.out[0]) a.out[0][row * a.ldo + col] = f32_to_bf16(gv);
          if (a.out[1]) a.out[1][row * a.ldo + col] = f32_to_bf16(uv);
          a.hraw[row * N + col] = f32_to_bf16(swiglu_value(gv, uv, a.gw ? a.gw[row] : 0.0f, a.gw != nullptr, a.limit));
        }
    } else {
      // SwiGLU of the bf16-rounded projections, then the fake quantization of each row's 128 outputs (the whole
      // workgroup: N % 128 == 0 is checked on the host) with the row's amax gathered over the 8 waves.
      __shared__ float red[W][16];
      float h[4], am[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * g + i;
        const float gv = round_bf16(acc[0][i]), uv = round_bf16(acc[NP - 1][i]);
        h[i] = 0.0f;
        if (r < M) {
          const size_t row = row0 + r, col = size_t(nt) * 16 + nl;
          if (a.out[0]) a.out[0][row * a.ldo + col] = f32_to_bf16(gv);
          if (a.out[1]) a.out[1][row * a.ldo + col] = f32_to_bf16(uv);
          h[i] = round_bf16(swiglu_value(gv, uv, a.gw ? a.gw[row] : 0.0f, a.gw != nullptr, a.limit));
        }
        am[i] = group_max<16>(fabsf(h[i]));
        if (nl == 0) red[wave][4 * g + i] = am[i];
      }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * g + i;
        if (r >= M) continue;
        const size_t row = row0 + r;
        if (a.gs_tab && !a.gs_tab[a.grow_expert[row]]) continue;
        float rm = red[0][r];
#pragma unroll
        for (int w = 1; w < W; ++w) rm = fmaxf(rm, red[w][r]);
        const Fp8Block blk = fp8_block_scale(rm);
        const size_t col = size_t(nt) * 16 + nl;
        const uint8_t c = fp8_code(h[i], blk);
        if (a.hh) a.hh[row * N + col] = f32_to_bf16(e4m3_to_f32(c) * blk.sc);
        if (a.hq) a.hq[row * N + col] = c;
        if (a.hs && wave == 0 && nl == 0) a.hs[row * (N / 128) + blockIdx.x] = blk.se;
      }
    }
  }
}

// Exhaustive decode check, one wave per e8m0 scale value sv (0..254): the scaled bf16 conversions of every e2m1 and
// e4m3 code (the bf16-MFMA kernels' dequantization), then the block-scaled MFMA's own decode. Weight operand: B[k][n] = e2m1 code
// (k/8 + n) % 16 with scale sv, activations one-hot 1.0 at k = 8m, so C[m][n] = e2m1((m+n) % 16) * 2^(sv-127).
// Activation operand: A[m][8m] = e4m3 code 16q + m (q = 0..15, 16 MFMAs) with scale sv, B all 1.0 (scale 127),
// so C[m][n] = e4m3(16q + m) * 2^(sv-127). Results are compared with the closed forms in fp32; cnt[0]
// counts mismatches where the expected value is a normal number, cnt[1] the compared normal values, cnt[2]
// mismatches at zero / subnormal / overflowing values (the hardware may flush those; no checkpoint scale
// produces them).
__device__ __forceinline__ void check_count(float got, float want, unsigned long long* c) {
  const float aw = fabsf(want);
  const bool normal = aw >= 1.17549435e-38f && aw <= 3.40282347e38f;
  const bool same = got == want;
  if (normal) {
    if (!same) atomicAdd(&c[0], 1ull);
    atomicAdd(&c[1], 1ull);
  } else if (aw != 0.0f && !same) {
    atomicAdd(&c[2], 1ull);
  }
}
// Sets the 8-bit operand byte of input k (0..127) to `code` in the lane of group (k % 64) / 16.
__device__ __forceinline__ void put_a8(v8i& a, int g, int k, int code) {
  if ((k % 64) / 16 != g) return;
  const int byte = (k / 64) * 16 + k % 16;
  a[byte / 4] |= code << (8 * (byte % 4));
}
// Exhaustive check of the hardware e4m3 encode (v_cvt_pk_fp8_f32: round to nearest even, OCP e4m3fn on gfx950)
// against f32_to_e4m3 on every fp32 value in [-448, 448] (both signs in one conversion), the domain every encoder
// here feeds it after clamping. cnt[0] += mismatching codes.
constexpr uint32_t kE4m3MaxBits = 0x43E00000u;  // 448.0f
__global__ __launch_bounds__(256) void fp8_check_encode_kernel(unsigned long long* cnt) {
  unsigned long long bad = 0;
  for (uint32_t u = blockIdx.x * 256u + threadIdx.x; u <= kE4m3MaxBits; u += gridDim.x * 256u) {
    const float x = __uint_as_float(u);
    const uint32_t hw = uint32_t(__builtin_amdgcn_cvt_pk_fp8_f32(x, -x, 0, false));
    bad += (hw & 0xffu) != f32_to_e4m3(x);
    bad += ((hw >> 8) & 0xffu) != f32_to_e4m3(-x);
  }
  if (bad) atomicAdd(&cnt[0], bad);
}

// Exhaustive check of the hardware bf16 rounding (v_cvt_pk_bf16_f32, what a float -> __bf16 conversion compiles to)
// against f32_to_bf16_sw on every fp32 bit pattern: cnt[0] += mismatches at non-NaN inputs, cnt[1] += at NaN inputs.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__global__ __launch_bounds__(256) void bf16_check_encode_kernel(unsigned long long* cnt) {
  unsigned long long bad = 0, bad_nan = 0;
  for (uint64_t u = blockIdx.x * 256ull + threadIdx.x; u < (1ull << 31); u += gridDim.x * 256ull) {
    const float x = __uint_as_float(uint32_t(u)), y = __uint_as_float(uint32_t(u) | 0x80000000u);
    const bf16x2_t v = {__bf16(x), __bf16(y)};
    const uint32_t hw = __builtin_bit_cast(uint32_t, v);
    const bool nan = (uint32_t(u) & 0x7fffffffu) > 0x7f800000u;
    if (nan) {  // a NaN must stay a NaN; differing payloads are counted apart
      bad += ((hw & 0x7fffu) <= 0x7f80u) + (((hw >> 16) & 0x7fffu) <= 0x7f80u);
      bad_nan += ((hw & 0xffffu) != f32_to_bf16_sw(x)) + ((hw >> 16) != f32_to_bf16_sw(y));
    } else {
      bad += ((hw & 0xffffu) != f32_to_bf16_sw(x)) + ((hw >> 16) != f32_to_bf16_sw(y));
    }
  }
  if (bad) atomicAdd(&cnt[0], bad);
  if (bad_nan) atomicAdd(&cnt[1], bad_nan);
}

__global__ __launch_bounds__(64) void mx_check_dequant_kernel(unsigned long long* cnt) {
  const int sv = blockIdx.x, lane = threadIdx.x, nl = lane & 15, g = lane >> 4;
  {  // weight side
    v8i a = {0, 0, 0, 0, 0, 0, 0, 0};
    put_a8(a, g, 8 * nl, 0x38);  // A[m][8m] = 1.0
    v4i b;
    for (int d = 0; d < 4; ++d) {
      uint32_t word = 0;
      for (int t = 0; t < 8; ++t) {
        const int k = 32 * g + 8 * d + t;
        word |= uint32_t((k / 8 + nl) % 16) << (4 * t);
      }
      b[d] = int(word);
    }
    const v4f c = mfma_fp8_fp4(a, b, 127, sv, v4f{0.0f, 0.0f, 0.0f, 0.0f});
    for (int i = 0; i < 4; ++i) {
      const int m = 4 * g + i;
      check_count(c[i], e2m1_to_f32(uint32_t((m + nl) % 16)) * e8m0_to_f32(uint8_t(sv)), cnt);
    }
  }
  {  // the scaled conversions used by the bf16 kernels: lane = byte value (x4), every code of the dword
    const float sc = e8m0_to_f32(uint8_t(sv));
    for (int rep = 0; rep < 4; ++rep) {
      const uint32_t byte = uint32_t(lane + 64 * rep);
      const uint32_t w = byte | (byte << 8) | (byte << 16) | (byte << 24);
      const bf16x8 d4 = fp4x8_to_bf16(w, sc);
      const bf16x8 d8 = fp8x8_to_bf16(w, w, sc);
      for (int i = 0; i < 8; ++i) {
        check_count(float(d4[i]), round_bf16(e2m1_to_f32((i & 1) ? (byte >> 4) : (byte & 15)) * sc), cnt);
        if ((byte & 0x7f) != 0x7f) check_count(float(d8[i]), round_bf16(e4m3_to_f32(uint8_t(byte)) * sc), cnt);
      }
    }
  }
  v4i ones;
  for (int d = 0; d < 4; ++d) ones[d] = 0x22222222;  // e2m1 code 2 = 1.0
  for (int q = 0; q < 16; ++q) {  // activation side
    const int code = 16 * q + nl;
    v8i a = {0, 0, 0, 0, 0, 0, 0, 0};
    put_a8(a, g, 8 * nl, code);
    const v4f c = mfma_fp8_fp4(a, ones, sv, 127, v4f{0.0f, 0.0f, 0.0f, 0.0f});
    for (int i = 0; i < 4; ++i) {
      const int cm = 16 * q + 4 * g + i;
      if ((cm & 0x7f) == 0x7f) continue;  // e4m3fn NaN codes
      check_count(c[i], e4m3_to_f32(uint8_t(cm)) * e8m0_to_f32(uint8_t(sv)), cnt);
    }
  }
}

template <class K>
void set_lds_limit(K kernel, size_t bytes) {
  if (bytes > 65536) UH_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                                  hipFuncAttributeMaxDynamicSharedMemorySize, int(bytes)));
}

static bool ksplit_enabled() {
  static const bool on = [] {
    const char* v = std::getenv("UH_GEMV_KSPLIT");
    return !v || std::string(v) != "0";
  }();
  return on;
}

// Workgroup shape: 8 waves (128 outputs) for every launch. A requantizing epilogue needs a whole 128-output block;
// for the others 8-wave workgroups measured 1% (decode) to 3% (verify) faster than 4-wave ones, whose smaller work
// items were expected to balance better.
template <int NP, int GM, int AM, int W>
void launch_gemv_w(const MxGemvArgs& a, int ntiles, hipStream_t st) {
  const size_t lds = size_t(a.rows_cap) * (a.K + GV_PAD) + size_t(a.rows_cap) * (a.K / 128);
  const size_t ntn = a.split ? size_t(a.split) : size_t(a.N) / 16;
  if constexpr (GM == 0 && NP == 1) {
    // A launch of fewer than 256 workgroups (one per CU) is latency-bound: split each tile's K over its waves.
    if (size_t(ntiles) * cdiv(ntn, W) < 256 && a.K % (128 * W) == 0 && !a.out32 && ksplit_enabled()) {
      auto* kern = &mx_gemv_kernel<NP, GM, AM, W, true>;
      set_lds_limit(kern, std::max<size_t>(lds, size_t(W) * NP * 64 * 16));
      kern<<<dim3(unsigned(ntn), unsigned(ntiles), 1), 64 * W, std::max<size_t>(lds, size_t(W) * NP * 64 * 16), st>>>(a);
      UH_CHECK_LAUNCH();
      return;
    }
  }
  const dim3 grid(cdiv(ntn, W), unsigned(ntiles), 1);
  // bf16 rows when they fit the LDS next to the epilogue's static share (the kernel's registers already hold it to
  // one 8-wave workgroup per CU)
  const size_t lds_bf = size_t(a.rows_cap + 1) * (a.K + 8) * 2;
  if (lds_bf <= 156 * 1024) {
    auto* kern = &mx_gemv_kernel<NP, GM, AM, W, false, true>;
    set_lds_limit(kern, lds_bf);
    kern<<<grid, 64 * W, lds_bf, st>>>(a);
    UH_CHECK_LAUNCH();
    return;
  }
  auto* kern = &mx_gemv_kernel<NP, GM, AM, W>;
  set_lds_limit(kern, lds);
  kern<<<grid, 64 * W, lds, st>>>(a);
  UH_CHECK_LAUNCH();
}
template <int NP, int GM, int AM>
void launch_gemv_t(const MxGemvArgs& a, int ntiles, hipStream_t st) {
  launch_gemv_w<NP, GM, AM, GV_WAVES>(a, ntiles, st);
}

// mx_xform_in_q (mx_moe.hip:132-176, kMode 1): rows r in [plan->remote0, plan->P) of a resident expert rebuilt from
// the compact fp8 token rows (quant_remote_tokens' codes q [U, K] and exponents qs [U, K / 128]) of token p2u[r].
// FP8 = false: xa[r] = bf16(e4m3 * 2^(e - 127)), exact with the scaled conversion (every such product is a bf16
// number), so bit-identical to mx_xform_in on the gathered rows; FP8 = true: the codes and exponents copied to the
// pair row (the MFMA operand form). 8 values per thread.
template <bool FP8>
__global__ __launch_bounds__(256) void mx_xform_q_kernel(const uint8_t* __restrict__ q, const uint8_t* __restrict__ qs,
                                                         const int32_t* __restrict__ p2u,
                                                         const MoePlan* __restrict__ plan,
                                                         const int32_t* __restrict__ row_expert,
                                                         const uint8_t* const* __restrict__ s_tab,
                                                         bf16* __restrict__ xa, uint8_t* __restrict__ qo,
                                                         uint8_t* __restrict__ qso, int K) {
  const int r0 = plan->remote0, per = K / 8, ks = K / 128;
  const size_t n = plan->P > r0 ? size_t(plan->P - r0) * per : 0;
  for (size_t it = blockIdx.x * size_t(blockDim.x) + threadIdx.x; it < n; it += size_t(gridDim.x) * blockDim.x) {
    const int r = r0 + int(it / per), c = int(it % per);
    if (s_tab && !s_tab[row_expert[r]]) continue;  // expert not on this device
    const size_t t = size_t(p2u[r]);
    const uint2 cc = *reinterpret_cast<const uint2*>(q + t * K + 8 * c);
    const uint8_t se = qs[t * ks + c / 16];
    if constexpr (FP8) {
      *reinterpret_cast<uint2*>(qo + size_t(r) * K + 8 * c) = cc;
      if ((c & 15) == 0) qso[size_t(r) * ks + c / 16] = se;
    } else {
      const bf16x8 v = fp8x8_to_bf16(cc.x, cc.y, e8m0_to_f32(se));
      *reinterpret_cast<bf16x8*>(xa + size_t(r) * K + 8 * c) = v;
    }
  }
}

}  // namespace

// ---- internal launchers (mx_internal.hpp) -----------------------------------------------------------------------------
static bool gemv_split_enabled() {
  static const bool on = [] {
    const char* v = std::getenv("UH_GEMV_SPLIT");
    return !v || std::string(v) != "0";
  }();
  return on;
}

void launch_mx_gemv(const MxGemvArgs& a, int ntiles, int amode, hipStream_t st) {
  if (ntiles <= 0) return;
  if (a.K % 128 || a.N % 16 || a.K <= 0 || a.N <= 0) throw std::runtime_error("mx_grouped_gemv: K % 128 or N % 16");
  if (a.rows_cap < 1 || a.rows_cap > GV_MAXROWS) throw std::runtime_error("mx_grouped_gemv: rows_cap");
  const bool np2 = a.w_tab[1] != nullptr, glu = a.hh || a.hq, graw = a.hraw != nullptr;
  if (glu && graw) throw std::runtime_error("mx_grouped_gemv: MxGlu h (raw) excludes hh / hq");
  if (graw && !np2) throw std::runtime_error("mx_grouped_gemv: glu needs two projections");
  if (glu && (!np2 || a.N % 128)) throw std::runtime_error("mx_grouped_gemv: glu needs two projections, N % 128");
  if (glu && a.hq && !a.hs) throw std::runtime_error("mx_grouped_gemv: glu hq without hs");
  if (amode ? !a.xa : (!a.aq || !a.as)) throw std::runtime_error("mx_grouped_gemv: null activations");
  if (amode == 2 && a.ldx % 8) throw std::runtime_error("mx_grouped_gemv: ldx % 8 (16-byte row loads)");
  if (!glu && !graw && ((!a.out[0] && !a.out32) || (np2 && !a.out[1])))
    throw std::runtime_error("mx_grouped_gemv: null output");
  if (!a.tiles) throw std::runtime_error("mx_grouped_gemv: null tiles");
#define UH_GV(NP, GLU)                                                       \
  (amode == 2   ? launch_gemv_t<NP, GLU, 2>(a, ntiles, st)                     \
   : amode == 1 ? launch_gemv_t<NP, GLU, 1>(a, ntiles, st)                     \
                : launch_gemv_t<NP, GLU, 0>(a, ntiles, st))
  if (glu) UH_GV(2, 1);
  else if (graw) UH_GV(2, 2);
  else if (np2) UH_GV(2, 0);
  else if (!a.out32 && a.N % 32 == 0 && size_t(ntiles) * cdiv(size_t(a.N) / 32, GV_WAVES) >= 512 &&
           gemv_split_enabled()) {
    // One matrix as two column streams per wave: twice the weight bytes behind each workgroup's start-up (the
    // staging of its rows and the first loads), half the workgroups -- when at least 512 remain (two per CU); a
    // smaller launch is latency-bound and wants every workgroup it can get.
    MxGemvArgs b = a;
    b.split = a.N / 32;
    b.w_tab[1] = a.w_tab[0];
    b.s_tab[1] = a.s_tab[0];
    b.out[1] = a.out[0] + a.N / 2;
    const MxGemvArgs& a = b;
    UH_GV(2, 0);
  } else UH_GV(1, 0);
#undef UH_GV
}

void launch_mx_transform(int mode, const bf16* x, int ldx, const int32_t* x_rows, const bf16* u, const float* w,
                         float limit, const int32_t* row_expert, const uint8_t* const* s_tab, bf16* out, uint8_t* q,
                         uint8_t* qs, int K, int P, hipStream_t st) {
  if (P <= 0) return;
  if (K % 128) throw std::runtime_error("mx transform: K % 128");
  if (ldx % 2) throw std::runtime_error("mx transform: ldx must be even (4-byte row pairs)");
  if (s_tab && !row_expert) throw std::runtime_error("mx transform: s_tab without row_expert");
  if (ldx % 8 == 0) {  // 16-byte rows: the 8-values-per-thread kernel
    const unsigned b8 = unsigned(std::min<size_t>((size_t(P) * (K / 8) + 255) / 256, 8192));
    if (mode == 2)
      mx_transform8_kernel<2><<<b8, 256, 0, st>>>(x, ldx, nullptr, u, ldx, w, limit, row_expert, s_tab, out, q, qs, K,
                                                  P);
    else
      mx_transform8_kernel<0><<<b8, 256, 0, st>>>(x, ldx, x_rows, nullptr, 0, nullptr, 0.0f, row_expert, s_tab, out, q,
                                                  qs, K, P);
    UH_CHECK_LAUNCH();
    return;
  }
  const unsigned blocks = transform_blocks(P, K);
  if (mode == 2)
    mx_transform_kernel<2><<<blocks, 256, 0, st>>>(x, ldx, nullptr, u, w, limit, row_expert, s_tab, out, q, qs, K, P);
  else if (out)
    mx_transform_kernel<0><<<blocks, 256, 0, st>>>(x, ldx, x_rows, nullptr, nullptr, 0.0f, row_expert, s_tab, out, q, qs, K, P);
  else
    mx_transform_kernel<1><<<blocks, 256, 0, st>>>(x, ldx, x_rows, nullptr, nullptr, 0.0f, row_expert, s_tab, nullptr, q, qs,
                                                   K, P);
  UH_CHECK_LAUNCH();
}

void launch_swiglu_quant(const bf16* g, int ldg, const bf16* u, int ldu, int M, int I, float limit, bf16* hh,
                         uint8_t* q, uint8_t* qs, hipStream_t st) {
  if (M <= 0) return;
  if (I % 128 || ldg % 8 || ldu % 8) throw std::runtime_error("swiglu quant: I % 128, ldg % 8, ldu % 8");
  const unsigned b8 = unsigned(std::min<size_t>((size_t(M) * (I / 8) + 255) / 256, 8192));
  mx_transform8_kernel<2><<<b8, 256, 0, st>>>(g, ldg, nullptr, u, ldu, nullptr, limit, nullptr, nullptr, hh, q, qs, I,
                                              M);
  UH_CHECK_LAUNCH();
}

// ---- public entry points ----------------------------------------------------------------------------------------------
void mx_repack_to(const uint8_t* w, const uint8_t* s, uint8_t* tw, uint8_t* ts, int N, int K, hipStream_t st) {
  if (N <= 0 || K <= 0 || N % 16 || K % 64) throw std::runtime_error("mx_repack_to: N % 16 or K % 64");
  mx_repack_kernel<<<cdiv(size_t(N) * (K / 32), 256), 256, 0, st>>>(w, s, tw, ts, N, K);
  UH_CHECK_LAUNCH();
}

void mx_repack(uint8_t* w, uint8_t* s, int N, int K, uint8_t* tmp, hipStream_t st) {
  const size_t wb = size_t(N) * K / 2, sb = size_t(N) * (K / 32);
  mx_repack_to(w, s, tmp, tmp + wb, N, K, st);
  UH_CHECK(hipMemcpyAsync(w, tmp, wb, hipMemcpyDeviceToDevice, st));
  UH_CHECK(hipMemcpyAsync(s, tmp + wb, sb, hipMemcpyDeviceToDevice, st));
}

void mx_xform_in(const bf16* x, int ldx, const int32_t* row_expert, const uint8_t* const* s_tab, bf16* xa, int P,
                 int K, hipStream_t st, const int32_t* x_rows) {
  launch_mx_transform(0, x, ldx, x_rows, nullptr, nullptr, 0.0f, row_expert, s_tab, xa, nullptr, nullptr, K, P, st);
}

void mx_xform_in_fp8(const bf16* x, int ldx, const int32_t* row_expert, const uint8_t* const* s_tab, uint8_t* q,
                     uint8_t* qs, int P, int K, hipStream_t st, const int32_t* x_rows) {
  if (!q || !qs) throw std::runtime_error("mx_xform_in_fp8: null q / qs");
  launch_mx_transform(1, x, ldx, x_rows, nullptr, nullptr, 0.0f, row_expert, s_tab, nullptr, q, qs, K, P, st);
}

namespace {
void launch_xform_q(bool fp8, const uint8_t* q, const uint8_t* s, const int32_t* p2u, const MoePlan* plan,
                    const int32_t* row_expert, const uint8_t* const* s_tab, bf16* xa, uint8_t* qo, uint8_t* qso, int P,
                    int K, hipStream_t st) {
  if (P <= 0) return;
  if (K <= 0 || K % 128) throw std::runtime_error("mx_xform_in_q: K % 128");
  if (!q || !s || !p2u || !plan || (s_tab && !row_expert)) throw std::runtime_error("mx_xform_in_q: null operand");
  if (reinterpret_cast<uintptr_t>(q) % 8) throw std::runtime_error("mx_xform_in_q: q not 8-byte aligned");
  if (fp8 ? (!qo || !qso || reinterpret_cast<uintptr_t>(qo) % 8) : (!xa || reinterpret_cast<uintptr_t>(xa) % 16))
    throw std::runtime_error("mx_xform_in_q: output null or misaligned");
  const unsigned blocks = unsigned(std::max<size_t>(1, std::min<size_t>((size_t(P) * (K / 8) + 255) / 256, 8192)));
  if (fp8)
    mx_xform_q_kernel<true><<<blocks, 256, 0, st>>>(q, s, p2u, plan, row_expert, s_tab, nullptr, qo, qso, K);
  else
    mx_xform_q_kernel<false><<<blocks, 256, 0, st>>>(q, s, p2u, plan, row_expert, s_tab, xa, nullptr, nullptr, K);
  UH_CHECK_LAUNCH();
}
}  // namespace

void mx_xform_in_q(const uint8_t* q, const uint8_t* s, const int32_t* p2u, const MoePlan* plan,
                   const int32_t* row_expert, const uint8_t* const* s_tab, bf16* xa, int P, int K, hipStream_t st) {
  launch_xform_q(false, q, s, p2u, plan, row_expert, s_tab, xa, nullptr, nullptr, P, K, st);
}
void mx_xform_in_q_fp8(const uint8_t* q, const uint8_t* s, const int32_t* p2u, const MoePlan* plan,
                       const int32_t* row_expert, const uint8_t* const* s_tab, uint8_t* qo, uint8_t* qso, int P, int K,
                       hipStream_t st) {
  launch_xform_q(true, q, s, p2u, plan, row_expert, s_tab, nullptr, qo, qso, P, K, st);
}

void mx_swiglu(const bf16* g, const bf16* u, const float* w, const int32_t* row_expert, const uint8_t* const* s_tab,
               bf16* hh, int P, int I, float limit, hipStream_t st) {
  launch_mx_transform(2, g, I, nullptr, u, w, limit, row_expert, s_tab, hh, nullptr, nullptr, I, P, st);
}

int mx_gemv_max_tokens() {
  static const int v = [] {
    const char* e = std::getenv("UNHOLY_MX_GEMV_TOKENS");
    return e ? std::max(kMxGemvTileRows, std::atoi(e)) : kMxGemvTileRows;
  }();
  return v;
}
// mx_grouped_gemm's small-tile route (max_rows <= 64 on the grouped GEMV); UNHOLY_MX_SKINNY=0 turns it off, as in the
// reference (mx_moe.hip:1033-1039).
bool mx_skinny_enabled() {
  static const bool on = [] {
    const char* v = std::getenv("UNHOLY_MX_SKINNY");
    return !(v && v[0] == '0' && v[1] == 0);
  }();
  return on;
}
bool mx_gemm_rb() { return false; }
void mx_gemm_force_rb(int) {}
void mx_gemm_rb_double_buffer(int) {}
namespace {
int g_glu = -1;
}
bool mx_gemm_glu() {
  static const bool env = [] {
    const char* v = std::getenv("UNHOLY_MX_GLU");
    return !v || std::string(v) != "0";
  }();
  return g_glu < 0 ? env : g_glu > 0;
}
void mx_gemm_force_glu(int on) { g_glu = on; }

unsigned long long fp8_check_encode(unsigned long long* total) {
  unsigned long long* cnt = nullptr;
  UH_CHECK(hipMalloc(&cnt, sizeof(unsigned long long)));
  UH_CHECK(hipMemset(cnt, 0, sizeof(unsigned long long)));
  fp8_check_encode_kernel<<<2048, 256>>>(cnt);
  UH_CHECK_LAUNCH();
  unsigned long long bad = 0;
  UH_CHECK(hipMemcpy(&bad, cnt, sizeof(bad), hipMemcpyDeviceToHost));
  UH_CHECK(hipFree(cnt));
  if (total) *total = 2ull * (kE4m3MaxBits + 1ull);
  return bad;
}

unsigned long long bf16_check_encode(unsigned long long* nan_bad) {
  unsigned long long* cnt = nullptr;
  UH_CHECK(hipMalloc(&cnt, 2 * sizeof(unsigned long long)));
  UH_CHECK(hipMemset(cnt, 0, 2 * sizeof(unsigned long long)));
  bf16_check_encode_kernel<<<4096, 256>>>(cnt);
  UH_CHECK_LAUNCH();
  unsigned long long h[2] = {};
  UH_CHECK(hipMemcpy(h, cnt, sizeof(h), hipMemcpyDeviceToHost));
  UH_CHECK(hipFree(cnt));
  if (nan_bad) *nan_bad = h[1];
  return h[0];
}

unsigned long long mx_check_dequant(unsigned long long* total) {
  unsigned long long* cnt = nullptr;
  UH_CHECK(hipMalloc(&cnt, 3 * sizeof(unsigned long long)));
  UH_CHECK(hipMemset(cnt, 0, 3 * sizeof(unsigned long long)));
  mx_check_dequant_kernel<<<255, 64>>>(cnt);
  UH_CHECK_LAUNCH();
  unsigned long long h[3] = {};
  UH_CHECK(hipMemcpy(h, cnt, sizeof(h), hipMemcpyDeviceToHost));
  UH_CHECK(hipFree(cnt));
  if (total) *total = h[1];
  return h[0];
}

namespace {
MxGemvArgs gemv_args(const bf16* xa, const uint8_t* q, const uint8_t* qs, int K, const Exl3Tile* tiles,
                     const uint8_t* const* w_tab, const uint8_t* const* s_tab, bf16* out, int ldo, int N,
                     const int* ntiles_dev, const uint8_t* const* w_tab2, const uint8_t* const* s_tab2, bf16* out2,
                     int rows_cap, const MxGlu& glu) {
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
  a.rows_cap = std::max(1, std::min(rows_cap, GV_MAXROWS));
  a.gw = glu.w;
  a.grow_expert = glu.row_expert;
  a.gs_tab = glu.s_tab;
  a.hh = glu.hh;
  a.hq = glu.hq;
  a.hs = glu.hs;
  a.hraw = glu.h;
  a.limit = glu.limit;
  if ((a.hh || a.hq || a.hraw) && a.gs_tab && !a.grow_expert) throw std::runtime_error("MxGlu: s_tab without row_expert");
  if (!w_tab || !s_tab) throw std::runtime_error("mx grouped: null tables");
  if (!w_tab2 != !s_tab2) throw std::runtime_error("mx grouped: second projection tables");
  return a;
}
}  // namespace

void mx_grouped_gemv(const bf16* xa, int K, const Exl3Tile* tiles, int ntiles, const uint8_t* const* w_tab,
                     const uint8_t* const* s_tab, bf16* out, int ldo, int N, hipStream_t st, const int* ntiles_dev,
                     const uint8_t* const* w_tab2, const uint8_t* const* s_tab2, bf16* out2, int max_rows,
                     const MxGlu& glu, const MxSums& sums) {
  if (sums.dst && (out2 || glu.hh || glu.hq || N % 128 || !sums.u2p || !sums.plan || sums.K <= 0))
    throw std::runtime_error("mx_grouped_gemv: sums shape");
  if ((glu.hh || glu.hq) && ldo != N) throw std::runtime_error("mx_grouped_gemv: glu shape (ldo != N)");
  launch_mx_gemv(gemv_args(xa, nullptr, nullptr, K, tiles, w_tab, s_tab, out, ldo, N, ntiles_dev, w_tab2, s_tab2,
                           out2, max_rows, glu),
                 ntiles, 1, st);
  // MxSums: each compact token's remote pair rows of out summed into sums.dst [U, N] (remote_combine's arithmetic),
  // as a second launch on the same stream; sums.counters are not used (the reference's are zero before and after).
  if (sums.dst && ntiles > 0)
    launch_remote_combine(out, ldo, sums.u2p, sums.plan, sums.dst, sums.K, N, 256, st);
}

void mx_grouped_gemv_q_f32out(const uint8_t* q, const uint8_t* qs, int K, const Exl3Tile* tiles, int ntiles,
                              const uint8_t* const* w_tab, const uint8_t* const* s_tab, float* out, int ldo, int N,
                              hipStream_t st, const int* ntiles_dev, int max_rows) {
  MxGemvArgs a = gemv_args(nullptr, q, qs, K, tiles, w_tab, s_tab, nullptr, ldo, N, ntiles_dev, nullptr, nullptr,
                           nullptr, max_rows, MxGlu{});
  a.out32 = out;
  launch_mx_gemv(a, ntiles, 0, st);
}

void mx_grouped_gemv_q(const uint8_t* q, const uint8_t* qs, int K, const Exl3Tile* tiles, int ntiles,
                       const uint8_t* const* w_tab, const uint8_t* const* s_tab, bf16* out, int ldo, int N,
                       hipStream_t st, const int* ntiles_dev, const uint8_t* const* w_tab2,
                       const uint8_t* const* s_tab2, bf16* out2, int max_rows, const MxGlu& glu) {
  if ((glu.hh || glu.hq) && ldo != N && (out || out2)) throw std::runtime_error("mx_grouped_gemv_q: glu shape");
  launch_mx_gemv(gemv_args(nullptr, q, qs, K, tiles, w_tab, s_tab, out, ldo, N, ntiles_dev, w_tab2, s_tab2, out2,
                           max_rows, glu),
                 ntiles, 0, st);
}

void mx_grouped_gemv_x(const bf16* x, int ldx, const int32_t* x_rows, int K, const Exl3Tile* tiles, int ntiles,
                       const uint8_t* const* w_tab, const uint8_t* const* s_tab, bf16* out, int ldo, int N,
                       hipStream_t st, const int* ntiles_dev, const uint8_t* const* w_tab2,
                       const uint8_t* const* s_tab2, bf16* out2, int max_rows, const MxGlu& glu) {
  if ((glu.hh || glu.hq) && ldo != N && (out || out2)) throw std::runtime_error("mx_grouped_gemv_x: glu shape");
  MxGemvArgs a = gemv_args(x, nullptr, nullptr, K, tiles, w_tab, s_tab, out, ldo, N, ntiles_dev, w_tab2, s_tab2, out2,
                           max_rows, glu);
  a.x_rows = x_rows;
  a.ldx = ldx;
  launch_mx_gemv(a, ntiles, 2, st);
}

}  // namespace unholy::kernels
