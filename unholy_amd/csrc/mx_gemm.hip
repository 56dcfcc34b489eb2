// Grouped MXFP4 GEMM for prefill tiles (up to 128 pair rows of one expert), and the dense fp8 GEMM dispatcher.
//
// Workgroup = one tile x 128 output columns (x 2 projections for w1 / w3 with the SwiGLU epilogue). Each wave owns a
// 64-row x 64-column block. Per 128-input stage the tile's activation rows are staged into LDS as bf16 (double
// buffered, the next stage's global loads in flight during the current stage's MFMAs), while every wave streams its
// own weight columns from HBM straight into registers (one stage ahead), dequantizes them exactly to bf16 and issues
// 32x32x16 bf16 MFMAs with fp32 accumulation. Weight columns are read from HBM once per tile; the activation tile is
// shared by the tile's column blocks, which the block mapping keeps on one XCD (one L2).
#include <algorithm>
#include <type_traits>
#include <cstdlib>

#include "common.hpp"
#include "numerics.hpp"
#include "unholy/kernels/mx_moe.hpp"
#include "mx_internal.hpp"
#include "fp8_internal.hpp"
#include "pipe.hpp"

namespace unholy::kernels {

using namespace uh;
using namespace pipe;

namespace {

constexpr int GM_BM = 128, GM_KS = 128, GM_LDA = GM_KS + 8;  // LDS row: 128 bf16 + 16 bytes of padding
constexpr size_t GM_ABUF = size_t(GM_BM) * GM_LDA * 2;       // one stage of A in LDS (bytes)

// The LDS A stage: row r holds inputs s*128 .. +127 of pair row row0 + r as bf16 (zeros past the tile's rows).
// Work item c of NT threads: row c / 8, inputs (c % 8) * 16 .. + 15 (16 values: 16 fp8 codes or 32 bytes of bf16).
template <int AM, int NT>
struct AStage {
  static constexpr int CH = GM_BM * 8 / NT;  // items per thread
  v4i raw[CH][AM == 0 ? 1 : 2];
  uint32_t sc[CH];

  // No branches around the loads (rows past the tile re-read its last row and are zeroed in store()): divergent
  // control flow here would make the compiler drain every outstanding load, the weight prefetch included.
  // Element offset of each item's row (loop-invariant: no dependent loads in the stage loop). Gathered rows (AM 2)
  // keep 64-bit offsets (row index x ldx can pass 2^32); the others are relative to the tile's first row (row0 K).
  std::conditional_t<AM == 2, size_t, uint32_t> rowoff[CH];
  size_t base = 0;

  __device__ __forceinline__ void rows(const MxGemvArgs& a, size_t row0, int M, int tid) {
    if constexpr (AM != 2) base = row0 * size_t(a.K);
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int r = min((tid + i * NT) / 8, M - 1);
      if constexpr (AM == 2) rowoff[i] = size_t(a.x_rows ? a.x_rows[row0 + r] : int(row0 + r)) * size_t(a.ldx);
      else rowoff[i] = uint32_t(r) * uint32_t(a.K);
    }
  }

  __device__ __forceinline__ void load(const MxGemvArgs& a, int s, int tid) {
    const auto qbase = as_global(a.aq + base + size_t(s) * GM_KS);  // AM 0 (uniform per stage)
    const auto xbase = as_global(a.xa + base + size_t(s) * GM_KS);  // AM 1, 2
    const auto sbase = as_global(a.as + base / 128 + size_t(s));    // AM 0: (row * K) / 128 = row * K/128
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const uint32_t part = uint32_t((tid + i * NT) % 8);
      if constexpr (AM == 0) {
        raw[i][0] = *reinterpret_cast<gptr<v4i>>(qbase + (rowoff[i] + part * 16));
        sc[i] = *(sbase + rowoff[i] / uint32_t(128));
      } else {
        raw[i][0] = *reinterpret_cast<gptr<v4i>>(xbase + (rowoff[i] + part * 16));
        raw[i][1] = *reinterpret_cast<gptr<v4i>>(xbase + (rowoff[i] + part * 16 + 8));
      }
    }
  }

  __device__ __forceinline__ void store(uint8_t* buf, int M, int tid) const {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = tid + i * NT, r = c / 8, part = c % 8;
      uint4 o0 = make_uint4(0, 0, 0, 0), o1 = o0;
      if constexpr (AM == 2) {  // act_quant of the raw row's 128-block: the 8 items of a row are 8 adjacent lanes
        float v[16], am = 0.0f;
        const uint32_t w[8] = {uint32_t(raw[i][0][0]), uint32_t(raw[i][0][1]), uint32_t(raw[i][0][2]),
                               uint32_t(raw[i][0][3]), uint32_t(raw[i][1][0]), uint32_t(raw[i][1][1]),
                               uint32_t(raw[i][1][2]), uint32_t(raw[i][1][3])};
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          v[2 * q] = __uint_as_float(w[q] << 16);
          v[2 * q + 1] = __uint_as_float(w[q] & 0xffff0000u);
        }
        if (r < M)
#pragma unroll
          for (int q = 0; q < 16; ++q) am = fmaxf(am, fabsf(v[q]));
        am = group_max<8>(am);
        if (r < M) {
          const Fp8Block blk = fp8_block_scale(am);
          uint32_t ow[8];
#pragma unroll
          for (int q = 0; q < 8; ++q)
            ow[q] = uint32_t(f32_to_bf16(e4m3_to_f32(fp8_code(v[2 * q], blk)) * blk.sc)) |
                    uint32_t(f32_to_bf16(e4m3_to_f32(fp8_code(v[2 * q + 1], blk)) * blk.sc)) << 16;
          o0 = make_uint4(ow[0], ow[1], ow[2], ow[3]);
          o1 = make_uint4(ow[4], ow[5], ow[6], ow[7]);
        }
      } else if (r < M) {
        if constexpr (AM == 0) {
          const float s = e8m0_to_f32(uint8_t(sc[i]));
          const bf16x8 lo = fp8x8_to_bf16(uint32_t(raw[i][0][0]), uint32_t(raw[i][0][1]), s);
          const bf16x8 hi = fp8x8_to_bf16(uint32_t(raw[i][0][2]), uint32_t(raw[i][0][3]), s);
          o0 = __builtin_bit_cast(uint4, lo);
          o1 = __builtin_bit_cast(uint4, hi);
        } else {
          o0 = __builtin_bit_cast(uint4, raw[i][0]);
          o1 = __builtin_bit_cast(uint4, raw[i][1]);
        }
      }
      uint8_t* dst = buf + (size_t(r) * GM_LDA + part * 16) * 2;
      *reinterpret_cast<uint4*>(dst) = o0;
      *reinterpret_cast<uint4*>(dst + 16) = o1;
    }
  }
};

// A wave's weight columns for one stage: 2 column blocks x 2 slabs of 64 inputs, 16 code bytes + 1 scale byte each.
struct BStage {
  v4i q[2][2];
  uint32_t s[2][2];
};

// NP 1: 4 waves = 2 row halves x 2 column halves (128 x 128); NP 2: 8 waves, the same for w1 (waves 0-3) and
// w3 (waves 4-7), with the SwiGLU + fake-quantization epilogue over the workgroup's 128 columns (one quant block).
template <int NP, int AM>
__global__ __launch_bounds__(256 * NP) void mx_gemm_kernel(MxGemvArgs a) {
  constexpr int NT = 256 * NP;
  extern __shared__ __align__(16) uint8_t smem[];
  // XCD-aware mapping: linear block ids go round-robin over the 8 XCDs; consecutive logical ids (the column blocks
  // of one tile, which read the same activation rows) are given to one XCD.
  int bx, by;
  tile_block(gridDim.x, bx, by);
  if (by >= a.ntiles || (a.ntiles_dev && by >= *a.ntiles_dev)) return;
  const Exl3Tile tile = a.tiles[by];
  if (tile.rows <= 0) return;
  const uint8_t* wps[NP];
  const uint8_t* sps[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    wps[p] = a.w_tab[p][tile.expert];
    sps[p] = a.s_tab[p][tile.expert];
    if (!wps[p] || !sps[p]) return;
  }
  const int K = a.K, N = a.N, KS = K / GM_KS, ntn = N / 16;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, h = lane >> 5;
  const int rh = wave & 1, chh = (wave >> 1) & 1, p = NP == 2 ? (wave >> 2) : 0;
  const uint8_t* wp = NP == 2 && p ? wps[NP - 1] : wps[0];
  const uint8_t* sp = NP == 2 && p ? sps[NP - 1] : sps[0];
  const int col0 = bx * 128 + chh * 64;  // the wave's first column
  // Per-lane weight offsets (column col0 + cb * 32 + l32, input half h of each 64-input slab).
  uint32_t cofs[2], sofs[2];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
    const int n = col0 + cb * 32 + l32;
    cofs[cb] = uint32_t((n / 16) * 512 + (n % 16) * 32 + h * 16);
    sofs[cb] = uint32_t((n / 16) * 32 + (n % 16) * 2 + h);
  }
  const size_t cslab = size_t(ntn) * 512, sslab = size_t(ntn) * 32;
  // The slab's base is uniform (scalar registers); the per-lane offset is loop-invariant: scalar-base loads with
  // no per-load address arithmetic and no 64-bit pointers kept live across the loop.
  const auto load_b = [&](BStage& b, int s) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const size_t kt = size_t(2 * s + j);
      const auto wbase = as_global(wp + kt * cslab);
      const auto sbase = as_global(sp + kt * sslab);
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        b.q[j][cb] = *reinterpret_cast<gptr<v4i>>(wbase + cofs[cb]);
        b.s[j][cb] = *(sbase + sofs[cb]);
      }
    }
  };

  for (int rg = 0; rg < tile.rows; rg += GM_BM) {
    const int M = min(GM_BM, tile.rows - rg);
    const size_t row0 = size_t(tile.row0) + rg;
    // 32-row blocks of this wave with rows (wave-uniform: a scalar value, so the MFMA guards are scalar branches)
    const int rb_live = __builtin_amdgcn_readfirstlane(min(2, max(0, (M - rh * 64 + 31) / 32)));
    v16f_t acc[2][2];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) acc[rb][cb] = v16f_t{};
    AStage<AM, NT> ast;
    BStage b2[2];
    __syncthreads();  // the previous row group's LDS reads are done
    ast.rows(a, row0, M, tid);
    ast.load(a, 0, tid);
    load_b(b2[0], 0);
    ast.store(smem, M, tid);
    lds_barrier();
    // One stage: prefetch stage s + 1 (activations into registers, weights into the other B buffer), MFMAs on
    // stage s, then the activations into the other LDS buffer. Unrolled by two so the B buffers do not move.
    const auto stage = [&](int s, BStage& bc, BStage& bn) {
      const uint8_t* abuf = smem + (s & 1) * GM_ABUF;
      const int sn = min(s + 1, KS - 1);
      if (s + 1 < KS) ast.load(a, sn, tid);
      load_b(bn, sn);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          // MFMA sub-step (j, t): both operands take inputs 64j + 32h + 8t .. + 7 of the stage.
          bf16x8 bf[2];
#pragma unroll
          for (int cb = 0; cb < 2; ++cb)
            bf[cb] = fp4x8_to_bf16(uint32_t(bc.q[j][cb][t]), __uint_as_float(bc.s[j][cb] << 23));
#pragma unroll
          for (int rb = 0; rb < 2; ++rb) {
            if (rb >= rb_live) break;
            const int r = rh * 64 + rb * 32 + l32;
            const bf16x8 af =
                *reinterpret_cast<const bf16x8*>(abuf + (size_t(r) * GM_LDA + 64 * j + 32 * h + 8 * t) * 2);
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) acc[rb][cb] = mfma32_bf16(af, bf[cb], acc[rb][cb]);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      if (s + 1 < KS) {
        ast.store(smem + ((s + 1) & 1) * GM_ABUF, M, tid);
        lds_barrier();
      }
    };
    for (int s = 0; s < KS; s += 2) {
      stage(s, b2[0], b2[1]);
      if (s + 1 < KS) stage(s + 1, b2[1], b2[0]);
    }

    // ---- epilogue, through LDS (the A buffers are free after the last stage): each wave writes its 64 x 64 block,
    // then the workgroup stores whole rows with 16-byte accesses. Value i of lane l of a 32 x 32 MFMA block sits at
    // row 8 (i/4) + 4 h + i % 4, column l32.
    __syncthreads();
    constexpr int LDC = 128 + 8;  // LDS row of the 128-column tile (bf16), padded
    uint16_t* sc = reinterpret_cast<uint16_t*>(smem);
    const auto put = [&](uint16_t* t, int rb, int cb, int i, uint16_t v) {
      t[(rh * 64 + rb * 32 + 8 * (i / 4) + 4 * h + (i % 4)) * LDC + chh * 64 + cb * 32 + l32] = v;
    };
    if constexpr (NP == 1) {
      if (a.out32) {  // fp32 rows: 128 x 128 x 4 bytes, each wave's block written and stored in turn by its lanes
        float* sf = reinterpret_cast<float*>(smem);
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
          for (int cb = 0; cb < 2; ++cb)
#pragma unroll
            for (int i = 0; i < 16; ++i)
              sf[(rh * 64 + rb * 32 + 8 * (i / 4) + 4 * h + (i % 4)) * 132 + chh * 64 + cb * 32 + l32] = acc[rb][cb][i];
        __syncthreads();
        for (int e = tid; e < M * 32; e += NT) {
          const int r = e / 32, c4 = (e % 32) * 4;
          *reinterpret_cast<float4*>(a.out32 + (row0 + r) * a.ldo + bx * 128 + c4) =
              *reinterpret_cast<const float4*>(sf + r * 132 + c4);
        }
      } else {
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
          for (int cb = 0; cb < 2; ++cb)
#pragma unroll
            for (int i = 0; i < 16; ++i) put(sc, rb, cb, i, f32_to_bf16(acc[rb][cb][i]));
        __syncthreads();
        for (int e = tid; e < M * 16; e += NT) {
          const int r = e / 16, c8 = (e % 16) * 8;
          *reinterpret_cast<uint4*>(a.out[0] + (row0 + r) * a.ldo + bx * 128 + c8) =
              *reinterpret_cast<const uint4*>(sc + r * LDC + c8);
        }
      }
    } else {
      // 1. w3 waves: bf16(u) into the tile. 2. w1 waves: h = bf16(SwiGLU(bf16(g), u)) over u in place. 3. the whole
      // workgroup: each row's amax and fake quantization of its 128 outputs (one block).
      if (p == 1)
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
          for (int cb = 0; cb < 2; ++cb)
#pragma unroll
            for (int i = 0; i < 16; ++i) put(sc, rb, cb, i, f32_to_bf16(acc[rb][cb][i]));
      __syncthreads();
      if (p == 0) {
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int r = rh * 64 + rb * 32 + 8 * (i / 4) + 4 * h + (i % 4);
            const float w = a.gw && r < M ? a.gw[row0 + r] : 0.0f;
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) {
              uint16_t* cell = sc + r * LDC + chh * 64 + cb * 32 + l32;
              const float gv = round_bf16(acc[rb][cb][i]);
              const uint16_t u = *cell;
              const float hval = swiglu_value(gv, bf16_to_f32(u), w, a.gw != nullptr, a.limit);
              if (r < M) {
                if (a.out[0]) a.out[0][(row0 + r) * a.ldo + col0 + cb * 32 + l32] = f32_to_bf16(gv);
                if (a.out[1]) a.out[1][(row0 + r) * a.ldo + col0 + cb * 32 + l32] = u;
              }
              *cell = f32_to_bf16(hval);
            }
          }
      }
      __syncthreads();
      // 16 consecutive threads take one row (8 outputs each): its amax is a DPP row max. The loop bound is
      // uniform, so every 16-lane group is whole; threads past the tile's rows only take part in the max.
      for (int e0 = 0; e0 < M * 16; e0 += NT) {
        const int e = e0 + tid, r = min(e / 16, M - 1), c8 = (e % 16) * 8;
        const uint4 hv = *reinterpret_cast<const uint4*>(sc + r * LDC + c8);
        const uint32_t hw[4] = {hv.x, hv.y, hv.z, hv.w};
        float am = 0.0f;
#pragma unroll
        for (int q = 0; q < 8; ++q) am = fmaxf(am, fabsf(bf16_to_f32(uint16_t(hw[q / 2] >> (16 * (q % 2))))));
        am = row16_max(am);
        const size_t row = row0 + r;
        if (e >= M * 16 || (a.gs_tab && !a.gs_tab[a.grow_expert[row]])) continue;
        const Fp8Block blk = fp8_block_scale(am);
        uint32_t qb[2] = {0, 0}, fq[4];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const uint8_t c = fp8_code(bf16_to_f32(uint16_t(hw[q / 2] >> (16 * (q % 2)))), blk);
          qb[q / 4] |= uint32_t(c) << (8 * (q % 4));
          const uint32_t f = f32_to_bf16(e4m3_to_f32(c) * blk.sc);
          fq[q / 2] = (q % 2) ? (fq[q / 2] | f << 16) : f;
        }
        const size_t o = row * N + size_t(bx) * 128 + c8;
        if (a.hq) *reinterpret_cast<uint2*>(a.hq + o) = make_uint2(qb[0], qb[1]);
        if (a.hh) *reinterpret_cast<uint4*>(a.hh + o) = make_uint4(fq[0], fq[1], fq[2], fq[3]);
        if (a.hs && c8 == 0) a.hs[row * (N / 128) + bx] = blk.se;
      }
    }
  }
}

// ---- Pipelined kernel for fp8 activation codes: an LDS ring filled by direct global -> LDS loads ----------------
//
// Workgroup = 256 threads (4 waves), one tile x 256 output columns: 128 columns each of w1 and w3 (NP 2, SwiGLU
// epilogue) or 256 columns of one matrix (NP 1). Wave w computes columns 64 w .. 64 w + 63 over all of the tile's
// rows: 4 x 2 MFMA blocks of 32 x 32, 3 conversions per MFMA. Per 128-input stage a ring slot holds
//   A  16 KB: the tile's fp8 codes, row r's 16-byte piece p at slot r * 8 + (p ^ lds_swz(r)) (conflict-free MFMA reads);
//   B  16 KB: 16 blocks of 1 KB = (projection or column half q, 64-input slab j, 32-column block c); slot h * 32 + n
//      of a block holds input half h (32 codes) of its column n, so a wave's operand read is 1 KB contiguous;
//   Bs  1 KB: the e8m0 weight scales of (q, j) in their global order (256 B each).
// Two slots (66 KB) plus the activation scales of all stages (copied once per row group) keep a workgroup within
// 80 KB of LDS, so two workgroups share a CU. Each has its own stage barriers: while one waits at a barrier or for
// its first operands, the other's MFMAs run. (One 8-wave workgroup per CU with a 4-slot ring stalled both waves of
// every SIMD at each barrier and measured 12-16% slower.) Every wave issues 4 A, 4 B and 1 scale load per stage;
// stage s + 1 is issued right after stage s's barrier, so only stage s is in flight when it is waited for. The loads
// are inline assembly: the compiler, seeing LDS written from global loads, would otherwise wait for every one of
// them before each LDS read.
constexpr int GP_A = 128 * 128, GP_B = 16 * 1024, GP_BS = 1024;
constexpr int GP_STAGE = GP_A + GP_B + GP_BS;
constexpr int GP_S = 2, GP_RING = GP_S * GP_STAGE;
constexpr int GP_MAX_KS = (80 * 1024 - GP_RING) / 128;  // activation scales [KS][128] after the ring
constexpr int GP_LDC1 = 256 + 8, GP_LDC2 = 128 + 8;
constexpr int GP_C1 = 128 * GP_LDC1 * 2, GP_C2 = 2 * 128 * GP_LDC2 * 2;
static_assert(GP_C1 <= GP_RING, "the bf16 C tile reuses the ring");
constexpr int GP_ROWS = 1024;  // the SwiGLU epilogue's per-row weights and flags, after the C tiles

// The bf16 / fp32 / SwiGLU epilogue of the pipelined kernels. each(f) calls f(row, column within the wave's 64, value)
// for every accumulator element; the ring is reused as the C tile.
template <int NP, class Each>
__device__ __forceinline__ void gp_epilogue(const MxGemvArgs& a, uint8_t* smem, int M, size_t row0, int bx, int cq,
                                            int tid, const Each& each) {
  const int N = a.N, q_own = cq >> 1;
  // ---- the ring is free once every wave is past its last stage
  __syncthreads();
  if constexpr (NP == 1) {
    const int c0 = cq * 64;
    if (a.out32) {  // fp32 outputs (accuracy checks): two passes of 64 rows through the ring
      constexpr int LDF = 256 + 4;
      static_assert(64 * LDF * 4 <= GP_RING, "a 64-row fp32 half tile fits the ring");
      float* sf = reinterpret_cast<float*>(smem);
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        if (half) __syncthreads();  // the first half's stores have read the tile
        each([&](int row, int col, float v) {
          if (row >= 64 * half && row < 64 * half + 64) sf[(row - 64 * half) * LDF + c0 + col] = v;
        });
        __syncthreads();
        for (int e = tid; e < min(64, M - 64 * half) * 64; e += 256) {
          const int r = e / 64, c4 = (e % 64) * 4;
          *reinterpret_cast<float4*>(a.out32 + (row0 + 64 * half + r) * a.ldo + bx * 256 + c4) =
              *reinterpret_cast<const float4*>(sf + r * LDF + c4);
        }
      }
    } else {
      uint16_t* sc = reinterpret_cast<uint16_t*>(smem);
      each([&](int row, int col, float v) { sc[row * GP_LDC1 + c0 + col] = f32_to_bf16(v); });
      __syncthreads();
      // 256 columns, or 128 in the last block of a matrix with N % 256 == 128 (bf16-row kernel only)
      const int p8 = min(256, N - bx * 256) / 8;
      for (int e = tid; e < M * p8; e += 256) {
        const int r = e / p8, c8 = (e % p8) * 8;
        *reinterpret_cast<uint4*>(a.out[0] + (row0 + r) * a.ldo + bx * 256 + c8) =
            *reinterpret_cast<const uint4*>(sc + r * GP_LDC1 + c8);
      }
    }
  } else {
    // bf16 g (w1) and u (w3) tiles in LDS, then 8 consecutive outputs of one row per thread: h = bf16(SwiGLU(g, u)),
    // the row's amax over its 128 outputs (16 threads: a DPP row max), fake quantization, 16-byte stores.
    // Each row's routing weight and whether its expert's w2 is here, loaded once per row (threads 0..127) into LDS
    // beside the tiles, so that the loop below has no dependent global loads.
    uint16_t* const tg = reinterpret_cast<uint16_t*>(smem);
    uint16_t* const tu = tg + 128 * GP_LDC2;
    uint16_t* const mine = q_own ? tu : tg;
    float* const rw_lds = reinterpret_cast<float*>(smem + GP_C2);
    int* const live_lds = reinterpret_cast<int*>(smem + GP_C2 + 512);
    float rw_t = 0.0f;
    int live_t = 1;
    if (tid < M) {
      const size_t row = row0 + tid;
      if (a.gw) rw_t = a.gw[row];
      if (a.gs_tab) live_t = a.gs_tab[a.grow_expert[row]] != nullptr;
    }
    const int chh = cq & 1;
    each([&](int row, int col, float v) { mine[row * GP_LDC2 + chh * 64 + col] = f32_to_bf16(v); });
    if (tid < 128) {
      rw_lds[tid] = rw_t;
      live_lds[tid] = live_t;
    }
    __syncthreads();
    for (int e0 = 0; e0 < M * 16; e0 += 256) {  // uniform bound: every 16-lane group is whole
      const int e = e0 + tid, r = min(e / 16, M - 1), c8 = (e % 16) * 8;
      const size_t row = row0 + r;
      const uint4 gv4 = *reinterpret_cast<const uint4*>(tg + r * GP_LDC2 + c8);
      const uint4 uv4 = *reinterpret_cast<const uint4*>(tu + r * GP_LDC2 + c8);
      const uint32_t gw4[4] = {gv4.x, gv4.y, gv4.z, gv4.w}, uw4[4] = {uv4.x, uv4.y, uv4.z, uv4.w};
      const float w = rw_lds[r];
      float hv[8], am = 0.0f;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        hv[q] = round_bf16(swiglu_value(bf16_to_f32(uint16_t(gw4[q / 2] >> (16 * (q % 2)))),
                                        bf16_to_f32(uint16_t(uw4[q / 2] >> (16 * (q % 2)))), w, a.gw != nullptr,
                                        a.limit));
        am = fmaxf(am, fabsf(hv[q]));
      }
      am = row16_max(am);
      if (e >= M * 16) continue;
      const size_t oc = row * a.ldo + size_t(bx) * 128 + c8;
      if (a.out[0]) *reinterpret_cast<uint4*>(a.out[0] + oc) = gv4;
      if (a.out[1]) *reinterpret_cast<uint4*>(a.out[1] + oc) = uv4;
      if (!live_lds[r]) continue;
      const Fp8Block blk = fp8_block_scale(am);
      uint32_t qb[2];
      fp8_codes8(hv, blk, qb[0], qb[1]);
      const size_t o = row * N + size_t(bx) * 128 + c8;
      if (a.hq) *reinterpret_cast<uint2*>(a.hq + o) = make_uint2(qb[0], qb[1]);
      if (a.hh)  // the fake-quantized rows (the codes decoded back, exact), only when asked for
        *reinterpret_cast<uint4*>(a.hh + o) = __builtin_bit_cast(uint4, fp8x8_to_bf16(qb[0], qb[1], blk.sc));
      if (a.hs && c8 == 0) a.hs[row * (N / 128) + bx] = blk.se;
    }
  }
}

template <int NP, bool SC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void mx_gemm_pipe_kernel(MxGemvArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  int bx, by;
  tile_block(gridDim.x, bx, by);
  if (by >= a.ntiles || (a.ntiles_dev && by >= *a.ntiles_dev)) return;
  const Exl3Tile tile = a.tiles[by];
  if (tile.rows <= 0) return;
  const uint8_t* wq[2];
  const uint8_t* sq[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    wq[q] = a.w_tab[NP == 2 ? q : 0][tile.expert];
    sq[q] = a.s_tab[NP == 2 ? q : 0][tile.expert];
    if (!wq[q] || !sq[q]) return;
  }
  const int K = a.K, KS = K / 128, N = a.N, ntn = N / 16;
  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // column quarter
  const int cq = wave, q_own = cq >> 1;
  const int colq0 = NP == 2 ? bx * 128 : bx * 256, colq_step = NP == 2 ? 0 : 128;
  const size_t cslab = size_t(ntn) * 512, sslab = size_t(ntn) * 32;
  const uint32_t lds0 = lds_addr(smem);
  uint8_t* const as_lds = smem + GP_RING;
  const uint32_t boff = uint32_t((l32 * 2 + h) * 16);  // B block: slot h*32+n <- piece 2n+h
  const int sc_q = wave >> 1, sc_j = wave & 1;         // this wave's 256-byte scale run (q, j)

  for (int rg = 0; rg < tile.rows; rg += 128) {
    const int M = min(128, tile.rows - rg);
    const size_t row0 = size_t(tile.row0) + rg;
    __syncthreads();  // the previous row group's LDS use is over
    // Each lane's A source in 16-byte units from a.aq (a gathered row's byte offset can pass 4 GiB).
    uint32_t a16[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int slot = (wave * 4 + i) * 64 + lane, r = slot >> 3, p = (slot & 7) ^ lds_swz(r);
      const int rr = min(r, M - 1);  // rows past the tile repeat its last
      a16[i] = uint32_t(a.x_rows ? a.x_rows[row0 + rr] : int(row0 + rr)) * uint32_t(K / 16) + uint32_t(p);
    }
    const auto issue = [&](int s) {
      const uint32_t st = __builtin_amdgcn_readfirstlane(lds0 + uint32_t((s % GP_S) * GP_STAGE));
#pragma unroll
      for (int i = 0; i < 4; ++i) dma16_g(a.aq + s * 128, a16[i], st + uint32_t(wave * 4 + i) * 1024);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int u = wave * 4 + i, q = u >> 3, j = (u >> 2) & 1, c = u & 3;
        const uint8_t* bb = wq[q] + size_t(2 * s + j) * cslab + size_t((colq0 + q * colq_step) / 16) * 512 + c * 1024;
        dma16_nt(bb, boff, st + uint32_t(GP_A + u * 1024));
      }
      const uint8_t* sb = sq[sc_q] + size_t(2 * s + sc_j) * sslab + size_t((colq0 + sc_q * colq_step) / 16) * 32;
      if (lane < 16) dma16(sb, uint32_t(lane) * 16, st + uint32_t(GP_A + GP_B + (sc_q * 2 + sc_j) * 256));
    };
    issue(0);
    {  // activation scales, after stage 0 is in flight (every thread keeps one row: 256 % 128 == 0). Row r of
       // stage s sits at s * 128 + (r % 16) * 8 + r / 16, so a lane's 8 row blocks are one 8-byte read.
      const int r = min(tid & 127, M - 1);
      const uint8_t* srow = a.as + size_t(a.x_rows ? a.x_rows[row0 + r] : int(row0 + r)) * KS;
      for (int e = tid; e < 128 * KS; e += 256) as_lds[(e & ~127) + (e & 15) * 8 + ((e >> 4) & 7)] = srow[e >> 7];
    }
    // The epilogue, given each(f): f(row, column in the wave's 64, value) for every accumulator element.

    // The K loop, specialised on the tile's live row blocks (RB): each stage is one basic block the compiler can
    // interleave, and only live accumulators exist (dead ones kept alive across the loop cost register copies in
    // every stage).
    const auto tile_body = [&](auto nrb) {
      constexpr int RB = decltype(nrb)::value;
      if constexpr (SC) {
        // Scaled MFMA 16x16x128 (fp8 x fp4, per-32 e8m0 scales in the instruction), 16-row blocks; no conversions.
        v4f acc[RB][4];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int cb = 0; cb < 4; ++cb) acc[rb][cb] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        const int m16 = lane & 15, g = lane >> 4, jb = g >> 1, hb = g & 1;
        for (int s = 0; s < KS; ++s) {
          wait_vm<0>();     // this wave's part of stage s (the only stage in flight)
          __syncthreads();  // every wave's part has landed; the other slot (stage s - 1) is free
          if (s + 1 < KS) issue(s + 1);
          const uint8_t* stb = smem + (s % GP_S) * GP_STAGE;
          v4i bq[4];
          int bsc[4];
#pragma unroll
          for (int cb = 0; cb < 4; ++cb) {  // column cq % 2 * 64 + 16 cb + m16, inputs 32 g .. 32 g + 31
            const int n = (cq & 1) * 64 + cb * 16 + m16, c = n >> 5;
            bq[cb] = *reinterpret_cast<const v4i*>(stb + GP_A + (q_own * 8 + jb * 4 + c) * 1024 + (hb * 32 + (n & 31)) * 16);
            bsc[cb] = stb[GP_A + GP_B + (q_own * 2 + jb) * 256 + (n >> 4) * 32 + (n & 15) * 2 + hb];
          }
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) {  // row 16 rb + m16: inputs 16 g .. + 15 and 64 + 16 g .. + 15
            const int r = rb * 16 + m16;
            const v4i lo = *reinterpret_cast<const v4i*>(stb + (r * 8 + (g ^ lds_swz(r))) * 16);
            const v4i hi = *reinterpret_cast<const v4i*>(stb + (r * 8 + ((4 + g) ^ lds_swz(r))) * 16);
            const v8i aq = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            const int asc = as_lds[s * 128 + m16 * 8 + rb];
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) acc[rb][cb] = mfma_fp8_fp4(aq, bq[cb], asc, bsc[cb], acc[rb][cb]);
          }
        }
        gp_epilogue<NP>(a, smem, M, row0, bx, cq, tid, [&](const auto& f) {
#pragma unroll
          for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int cb = 0; cb < 4; ++cb)
#pragma unroll
              for (int i = 0; i < 4; ++i) f(rb * 16 + 4 * g + i, cb * 16 + m16, acc[rb][cb][i]);
        });
      } else {
        // Exact dequantization + bf16 MFMA 16x16x32, 16-row blocks: one MFMA per 32-input block, so every output
        // accumulates acc + (block sum) x (scales) block after block in input order, as the reference's fma chain
        // over the block and fold (ref_gemm.hip:54-63) does. The block's 32 products are exact (e4m3 x 2^a and
        // e2m1 x 2^w are bf16 numbers), their sum is exact in fp32 for the activation blocks act_quant produces,
        // and the MFMA adds it to the accumulator with one rounding: the same fp32 value as the reference order.
        // Lane (row or column l % 16, g = l / 16) holds inputs 8g .. 8g + 7 of the block on both sides.
        //
        // Software pipelined: a stage's B words, B scales and A scales are read right after its barrier, and the A
        // pieces of block b + 1 are read while block b's conversions and MFMAs run, so LDS latency is hidden
        // behind 4 x RB MFMAs instead of being waited for before each row block.
        v4f acc[RB][4];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int cb = 0; cb < 4; ++cb) acc[rb][cb] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        const int m16 = lane & 15, g = lane >> 4;
        // A piece of row rb * 16 + m16 for block b: byte (a_lane ^ (b << 5)) + rb * 2048 of the stage. The swizzle
        // lds_swz(r) depends on m16 only (rb * 16 >> 1 is a multiple of 8), and piece 2b + (g >> 1) = 2b ^ (g >> 1).
        const uint32_t a_lane =
            uint32_t(m16 * 128 + (((g >> 1) ^ lds_swz(m16)) << 4) + (g & 1) * 8);
        // B word of column block cb, block b = 2j + h: byte b_lane + j * 4096 + (cb >> 1) * 1024 + h * 512 +
        // (cb & 1) * 256 of the stage; its scales (both h of slab j) the u16 at s_lane + j * 256 + cb * 32.
        const uint32_t b_lane = uint32_t(GP_A + q_own * 8192 + (cq & 1) * 2048 + m16 * 16 + 4 * g);
        const uint32_t s_lane = uint32_t(GP_A + GP_B + q_own * 512 + (cq & 1) * 128 + m16 * 2);
        for (int s = 0; s < KS; ++s) {
          wait_vm<0>();     // this wave's part of stage s (the only stage in flight)
          __syncthreads();  // every wave's part has landed; the other slot (stage s - 1) is free
          if (s + 1 < KS) issue(s + 1);
          const uint8_t* stb = smem + (s % GP_S) * GP_STAGE;
          const uint2 asw = *reinterpret_cast<const uint2*>(as_lds + s * 128 + m16 * 8);
          uint32_t bsc[2][4], bw[4][4];
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int cb = 0; cb < 4; ++cb)
              bsc[j][cb] = *reinterpret_cast<const uint16_t*>(stb + s_lane + j * 256 + cb * 32);
#pragma unroll
          for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int cb = 0; cb < 4; ++cb)
              bw[b][cb] = *reinterpret_cast<const uint32_t*>(stb + b_lane + (b >> 1) * 4096 + (cb >> 1) * 1024 +
                                                             (b & 1) * 512 + (cb & 1) * 256);
          uint2 araw[2][RB];
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) araw[0][rb] = *reinterpret_cast<const uint2*>(stb + a_lane + rb * 2048);
          float asc[RB];
#pragma unroll
          for (int rb = 0; rb < RB; ++rb)
            asc[rb] = __uint_as_float((((rb < 4 ? asw.x : asw.y) >> (8 * (rb & 3))) & 0xffu) << 23);
          __builtin_amdgcn_sched_barrier(0);  // the stage's reads all issued before any use
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            if (b < 3) {
#pragma unroll
              for (int rb = 0; rb < RB; ++rb)
                araw[(b + 1) & 1][rb] =
                    *reinterpret_cast<const uint2*>(stb + (a_lane ^ uint32_t((b + 1) << 5)) + rb * 2048);
            }
            __builtin_amdgcn_sched_barrier(0);  // keep the reads of block b + 1 ahead of block b's MFMAs
            bf16x8 bf[4];
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) {
              bf[cb] = fp4x8_to_bf16(bw[b][cb], __uint_as_float(((bsc[b >> 1][cb] >> (8 * (b & 1))) & 0xffu) << 23));
            }
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
              const uint2 av = araw[b & 1][rb];
              const bf16x8 af = fp8x8_to_bf16(av.x, av.y, asc[rb]);
#pragma unroll
              for (int cb = 0; cb < 4; ++cb) acc[rb][cb] = mfma_bf16(af, bf[cb], acc[rb][cb]);
            }
          }
        }
        gp_epilogue<NP>(a, smem, M, row0, bx, cq, tid, [&](const auto& f) {
#pragma unroll
          for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int cb = 0; cb < 4; ++cb)
#pragma unroll
              for (int i = 0; i < 4; ++i) f(rb * 16 + 4 * g + i, cb * 16 + m16, acc[rb][cb][i]);
        });
      }
    };
    {
      const int rb16 = __builtin_amdgcn_readfirstlane((M + 15) / 16);
      if (rb16 == 8) tile_body(std::integral_constant<int, 8>{});
      else if (rb16 == 7) tile_body(std::integral_constant<int, 7>{});
      else if (rb16 == 6) tile_body(std::integral_constant<int, 6>{});
      else if (rb16 == 5) tile_body(std::integral_constant<int, 5>{});
      else if (rb16 == 4) tile_body(std::integral_constant<int, 4>{});
      else if (rb16 == 3) tile_body(std::integral_constant<int, 3>{});
      else if (rb16 == 2) tile_body(std::integral_constant<int, 2>{});
      else tile_body(std::integral_constant<int, 1>{});
    }
  }
}


// ---- Pipelined kernel for bf16 activation rows (exact e4m3 x 2^k values, the fake-quantized rows of mx_xform_in) ----
//
// The same workgroup shape as mx_gemm_pipe_kernel (256 threads, one tile x 256 output columns, wave w owns columns
// 64 w .. 64 w + 63 over all rows, 16x16x32 bf16 MFMAs, one per 32-input block), but the activations arrive as bf16:
// they go from LDS straight into the MFMA with no conversion, and only the weights are dequantized (half a
// conversion per MFMA instead of one and a half). Stages are 64 inputs, three ring slots of 24.5 KB (73.5 KB, two
// workgroups per CU), two stages in flight. Per stage a slot holds
//   A  16 KB: 128 rows x 64 bf16, row r's 16-byte piece p at slot r * 8 + (p ^ lds_swz(r));
//   B   8 KB: 8 blocks of 1 KB = (projection or column half q, 32-column block c), slot h * 32 + n <- piece 2n + h;
//   Bs 512 B: the e8m0 weight scales of projection q at q * 256 in their global order.
// Every wave issues 4 A, 2 B and 1 scale load per stage (7 vm operations).
constexpr int kSkinnyMaxRows = 64;  // mx_grouped_gemm's max_rows bound for the GEMV route
constexpr int GB_KS = 64, GB_A = 128 * 128, GB_B = 8 * 1024, GB_BS = 512;
constexpr int GB_STAGE = GB_A + GB_B + GB_BS;
constexpr int GB_S = 3, GB_RING = GB_S * GB_STAGE;
static_assert(GP_C1 <= GB_RING && GP_C2 + GP_ROWS <= GB_RING && 64 * (256 + 4) * 4 <= GB_RING,
              "the C tiles reuse the ring");

template <int NP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void mx_gemm_pipe_bf16_kernel(MxGemvArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  int bx, by;
  tile_block(gridDim.x, bx, by);
  if (by >= a.ntiles || (a.ntiles_dev && by >= *a.ntiles_dev)) return;
  const Exl3Tile tile = a.tiles[by];
  if (tile.rows <= 0) return;
  const uint8_t* wq[2];
  const uint8_t* sq[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    wq[q] = a.w_tab[NP == 2 ? q : 0][tile.expert];
    sq[q] = a.s_tab[NP == 2 ? q : 0][tile.expert];
    if (!wq[q] || !sq[q]) return;
  }
  const int K = a.K, KS = K / GB_KS, N = a.N, ntn = N / 16;
  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // column quarter
  const int cq = wave, q_own = cq >> 1;
  // NP 1: columns bx 256 .. + 255 as two 128-column halves; the last block of a matrix with N % 256 == 128 has only
  // the first half, and its second-half waves stream that half again (their results are not stored).
  const int colq0 = NP == 2 ? bx * 128 : bx * 256, colq_step = NP == 2 || colq0 + 128 >= N ? 0 : 128;
  const size_t cslab = size_t(ntn) * 512, sslab = size_t(ntn) * 32;
  const uint32_t lds0 = lds_addr(smem);
  const uint32_t boff = uint32_t((l32 * 2 + h) * 16);  // B block: slot h*32+n <- piece 2n+h
  const int m16 = lane & 15, g = lane >> 4;
  // A piece of row rb * 16 + m16, inputs 32 b + 8 g .. + 7 (piece 4b + g): byte a_lane[b] + rb * 2048 of the stage
  // (lds_swz(rb * 16 + m16) == lds_swz(m16)).
  const uint32_t a_lane0 = uint32_t(m16 * 128 + ((g ^ lds_swz(m16)) << 4));
  const uint32_t a_lane1 = uint32_t(m16 * 128 + (((4 + g) ^ lds_swz(m16)) << 4));
  // B word of column block cb, block b: byte b_lane + (cb >> 1) * 1024 + b * 512 + (cb & 1) * 256; the two scales
  // of column block cb (b = 0, 1) the u16 at s_lane + cb * 32.
  const uint32_t b_lane = uint32_t(GB_A + q_own * 4096 + (cq & 1) * 2048 + m16 * 16 + 4 * g);
  const uint32_t s_lane = uint32_t(GB_A + GB_B + q_own * 256 + (cq & 1) * 128 + m16 * 2);

  for (int rg = 0; rg < tile.rows; rg += 128) {
    const int M = min(128, tile.rows - rg);
    const size_t row0 = size_t(tile.row0) + rg;
    __syncthreads();  // the previous row group's LDS use is over
    // Each lane's A source in 16-byte units from a.xa (a gathered row's byte offset can pass 4 GiB).
    uint32_t a16[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int slot = (wave * 4 + i) * 64 + lane, r = slot >> 3, p = (slot & 7) ^ lds_swz(r);
      const int rr = min(r, M - 1);  // rows past the tile repeat its last
      a16[i] = uint32_t(a.x_rows ? a.x_rows[row0 + rr] : int(row0 + rr)) * uint32_t(K / 8) + uint32_t(p);
    }
    const auto issue = [&](int s) {
      const uint32_t st = __builtin_amdgcn_readfirstlane(lds0 + uint32_t((s % GB_S) * GB_STAGE));
#pragma unroll
      for (int i = 0; i < 4; ++i) dma16_g(a.xa + s * 64, a16[i], st + uint32_t(wave * 4 + i) * 1024);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int u = wave * 2 + i, q = u >> 2, c = u & 3;
        const uint8_t* bb = wq[q] + size_t(s) * cslab + size_t((colq0 + q * colq_step) / 16) * 512 + c * 1024;
        dma16_nt(bb, boff, st + uint32_t(GB_A + u * 1024));
      }
      {  // scales: wave w copies bytes 128 w .. + 127 (projection w / 2), 8 lanes of 16 bytes
        const int q = wave >> 1;
        const uint8_t* sb = sq[q] + size_t(s) * sslab + size_t((colq0 + q * colq_step) / 16) * 32 + (wave & 1) * 128;
        if (lane < 8) dma16(sb, uint32_t(lane) * 16, st + uint32_t(GB_A + GB_B + wave * 128));
      }
    };
    issue(0);
    if (KS > 1) issue(1);

    const auto tile_body = [&](auto nrb) {
      constexpr int RB = decltype(nrb)::value;
      v4f acc[RB][4];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) acc[rb][cb] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
      for (int s = 0; s < KS; ++s) {
        if (s + 1 < KS) wait_vm<7>();  // stage s has landed; stage s + 1 may still be in flight
        else wait_vm<0>();
        __syncthreads();  // every wave's part of stage s has landed; slot (s + 2) % 3 (stage s - 1) is free
        if (s + 2 < KS) issue(s + 2);
        const uint8_t* stb = smem + (s % GB_S) * GB_STAGE;
        uint32_t bsc[4], bw[2][4];
        bf16x8 af[2][RB];
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) bsc[cb] = *reinterpret_cast<const uint16_t*>(stb + s_lane + cb * 32);
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
          for (int cb = 0; cb < 4; ++cb)
            bw[b][cb] = *reinterpret_cast<const uint32_t*>(stb + b_lane + (cb >> 1) * 1024 + b * 512 + (cb & 1) * 256);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) af[0][rb] = *reinterpret_cast<const bf16x8*>(stb + a_lane0 + rb * 2048);
        __builtin_amdgcn_sched_barrier(0);  // the stage's first reads all issued before any use
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) af[1][rb] = *reinterpret_cast<const bf16x8*>(stb + a_lane1 + rb * 2048);
        __builtin_amdgcn_sched_barrier(0);  // block 1's A reads issued ahead of block 0's MFMAs
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          bf16x8 bf[4];
#pragma unroll
          for (int cb = 0; cb < 4; ++cb)
            bf[cb] = fp4x8_to_bf16(bw[b][cb], __uint_as_float(((bsc[cb] >> (8 * b)) & 0xffu) << 23));
#pragma unroll
          for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) acc[rb][cb] = mfma_bf16(af[b][rb], bf[cb], acc[rb][cb]);
        }
      }
      gp_epilogue<NP>(a, smem, M, row0, bx, cq, tid, [&](const auto& f) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int cb = 0; cb < 4; ++cb)
#pragma unroll
            for (int i = 0; i < 4; ++i) f(rb * 16 + 4 * g + i, cb * 16 + m16, acc[rb][cb][i]);
      });
    };
    {
      const int rb16 = __builtin_amdgcn_readfirstlane((M + 15) / 16);
      if (rb16 == 8) tile_body(std::integral_constant<int, 8>{});
      else if (rb16 == 7) tile_body(std::integral_constant<int, 7>{});
      else if (rb16 == 6) tile_body(std::integral_constant<int, 6>{});
      else if (rb16 == 5) tile_body(std::integral_constant<int, 5>{});
      else if (rb16 == 4) tile_body(std::integral_constant<int, 4>{});
      else if (rb16 == 3) tile_body(std::integral_constant<int, 3>{});
      else if (rb16 == 2) tile_body(std::integral_constant<int, 2>{});
      else tile_body(std::integral_constant<int, 1>{});
    }
  }
}

template <int NP>
void launch_pipe_t(const MxGemvArgs& a, int ntiles, hipStream_t st) {
  const size_t lds = std::max<size_t>(size_t(GP_RING) + size_t(128) * (a.K / 128), NP == 2 ? GP_C2 + GP_ROWS : GP_C1);
  auto* kern = mx_gemm_exact() ? &mx_gemm_pipe_kernel<NP, false> : &mx_gemm_pipe_kernel<NP, true>;
  UH_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                               int(lds)));
  MxGemvArgs b = a;
  b.ntiles = ntiles;
  kern<<<tile_grid(a.N / (NP == 2 ? 128 : 256), ntiles), 256, lds, st>>>(b);
  UH_CHECK_LAUNCH();
}

template <int NP>
void launch_pipe_bf16_t(const MxGemvArgs& a, int ntiles, hipStream_t st) {
  const size_t lds = GB_RING;
  auto* kern = &mx_gemm_pipe_bf16_kernel<NP>;
  UH_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                               int(lds)));
  MxGemvArgs b = a;
  b.ntiles = ntiles;
  kern<<<tile_grid(NP == 2 ? a.N / 128 : (a.N + 255) / 256, ntiles), 256, lds, st>>>(b);
  UH_CHECK_LAUNCH();
}

template <int NP, int AM>
void launch_gemm_t(const MxGemvArgs& a, int ntiles, hipStream_t st) {
  const size_t lds = 2 * GM_ABUF;
  auto* kern = &mx_gemm_kernel<NP, AM>;
  UH_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                               int(lds)));
  MxGemvArgs b = a;
  b.ntiles = ntiles;
  kern<<<tile_grid(a.N / 128, ntiles), 256 * NP, lds, st>>>(b);
  UH_CHECK_LAUNCH();
}

}  // namespace

// UH_GEMM_PIPE=0 selects the register-staged kernel for fp8 codes too (comparison runs).
static bool pipe_disabled() {
  static const bool off = [] {
    const char* e = std::getenv("UH_GEMM_PIPE");
    return e && e[0] == '0';
  }();
  return off;
}


void launch_mx_gemm(const MxGemvArgs& a, int ntiles, int amode, hipStream_t st) {
  if (ntiles <= 0) return;
  // bf16 activation rows (amode 1) take the 64-input-stage pipelined kernel: K % 64 as the reference asks
  // (mx_moe.hip:1045); the other kernels stage 128 inputs at a time.
  const bool pipe16 = amode == 1 && !pipe_disabled() && a.N % 128 == 0 && a.K % GB_KS == 0 && !a.out32;
  if (a.K <= 0 || a.N <= 0 || a.N % 128 || (!pipe16 && a.K % GM_KS))
    throw std::runtime_error("mx_grouped_gemm: K % 128 (K % 64 for bf16 rows) or N % 128");
  const bool np2 = a.w_tab[1] != nullptr, glu = a.hh || a.hq;
  if (np2 && !glu) {  // two projections without the epilogue: one launch each
    MxGemvArgs b = a;
    b.w_tab[1] = nullptr;
    b.s_tab[1] = nullptr;
    b.out[1] = nullptr;
    launch_mx_gemm(b, ntiles, amode, st);
    b.w_tab[0] = a.w_tab[1];
    b.s_tab[0] = a.s_tab[1];
    b.out[0] = a.out[1];
    b.out32 = nullptr;
    launch_mx_gemm(b, ntiles, amode, st);
    return;
  }
  if (glu && !np2) throw std::runtime_error("mx_grouped_gemm: glu needs two projections");
  if (glu && a.hq && !a.hs) throw std::runtime_error("mx_grouped_gemm: glu hq without hs");
  if (!glu && !a.out[0] && !a.out32) throw std::runtime_error("mx_grouped_gemm: null output");
  if (amode ? !a.xa : (!a.aq || !a.as)) throw std::runtime_error("mx_grouped_gemm: null activations");
  if (amode == 2 && a.ldx % 8) throw std::runtime_error("mx_grouped_gemm: ldx % 8");
  if (!a.tiles) throw std::runtime_error("mx_grouped_gemm: null tiles");
  if ((a.out[0] || a.out[1]) && a.ldo % 8) throw std::runtime_error("mx_grouped_gemm: ldo % 8 (16-byte row stores)");
#define UH_GM(NP)                                                      \
  (amode == 2   ? launch_gemm_t<NP, 2>(a, ntiles, st)                   \
   : amode == 1 ? launch_gemm_t<NP, 1>(a, ntiles, st)                   \
                : launch_gemm_t<NP, 0>(a, ntiles, st))
  const bool pipe = amode == 0 && a.K / GM_KS <= GP_MAX_KS && !pipe_disabled();
  if (amode == 0 && a.x_rows && (!pipe || (!glu && a.N % 256)))
    throw std::runtime_error("mx_grouped_gemm_q: x_rows needs the pipelined kernel (K <= 14336, N % 256 without glu)");
  if (pipe16) {
    if (glu) launch_pipe_bf16_t<2>(a, ntiles, st);
    else launch_pipe_bf16_t<1>(a, ntiles, st);
  } else if (glu) {
    if (pipe) launch_pipe_t<2>(a, ntiles, st);
    else UH_GM(2);
  } else {
    if (pipe && a.N % 256 == 0) launch_pipe_t<1>(a, ntiles, st);
    else UH_GM(1);
  }
#undef UH_GM
}

void launch_fp8_gemm(const Fp8GemmArgs& a, hipStream_t st) {
  if (a.M > 0 && a.ldc < a.N) throw std::runtime_error("fp8 gemm: ldc < N");
  if (fp8_rows_fits(a)) launch_fp8_rows(a, st);
  else if (a.M <= 64) launch_fp8_gemv(a, st);
  else if (fp8_tiled_fits(a)) launch_fp8_tiled(a, st);
  else launch_fp8_skinny(a, st);
}

namespace {
MxGemvArgs gemm_args(const bf16* xa, const uint8_t* q, const uint8_t* qs, int K, const Exl3Tile* tiles,
                     const uint8_t* const* w_tab, const uint8_t* const* s_tab, bf16* out, int ldo, int N,
                     const int* ntiles_dev, const uint8_t* const* w_tab2, const uint8_t* const* s_tab2, bf16* out2,
                     const MxGlu& glu) {
  if (!w_tab || !s_tab) throw std::runtime_error("mx_grouped_gemm: null tables");
  if (glu.h) throw std::runtime_error("mx_grouped_gemm: MxGlu h (raw rows) is a GEMV option");
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

// max_rows: the caller's bound on any tile's rows (the reference's verify steps pass the step's token count, an expert
// having at most one row per token). Up to 64 rows (and K % 128) the tiles take the grouped GEMV in groups of up to
// 16 rows, each group streaming the tile's weights once, instead of a 128-row GEMM tile that is mostly padding: the
// same per-output arithmetic (every 32-input block's exact sum added to the fp32 accumulator in input order), so the
// outputs are the GEMM's bit for bit. Larger bounds, or K % 128 != 0, take the GEMM.
void mx_grouped_gemm(const bf16* xa, int K, const Exl3Tile* tiles, int ntiles, const uint8_t* const* w_tab,
                     const uint8_t* const* s_tab, bf16* out, int ldo, int N, hipStream_t st, const int* ntiles_dev,
                     const uint8_t* const* w_tab2, const uint8_t* const* s_tab2, bf16* out2, int max_rows) {
  MxGemvArgs a = gemm_args(xa, nullptr, nullptr, K, tiles, w_tab, s_tab, out, ldo, N, ntiles_dev, w_tab2, s_tab2, out2,
                           MxGlu{});
  if (max_rows >= 1 && max_rows <= kSkinnyMaxRows && K % 128 == 0 && K > 0 && N % 16 == 0 && mx_skinny_enabled()) {
    a.rows_cap = std::min(max_rows, 16);
    launch_mx_gemv(a, ntiles, 1, st);
    return;
  }
  launch_mx_gemm(a, ntiles, 1, st);
}

void mx_grouped_gemm_q(const uint8_t* q, const uint8_t* qs, int K, const Exl3Tile* tiles, int ntiles,
                       const uint8_t* const* w_tab, const uint8_t* const* s_tab, bf16* out, int ldo, int N,
                       hipStream_t st, const int* ntiles_dev, const uint8_t* const* w_tab2,
                       const uint8_t* const* s_tab2, bf16* out2, int, const MxGlu& glu, const int32_t* x_rows) {
  MxGemvArgs a = gemm_args(nullptr, q, qs, K, tiles, w_tab, s_tab, out, ldo, N, ntiles_dev, w_tab2, s_tab2, out2, glu);
  a.x_rows = x_rows;
  launch_mx_gemm(a, ntiles, 0, st);
}

void mx_grouped_gemm_q_f32out(const uint8_t* q, const uint8_t* qs, int K, const Exl3Tile* tiles, int ntiles,
                              const uint8_t* const* w_tab, const uint8_t* const* s_tab, float* out, int ldo, int N,
                              hipStream_t st, const int* ntiles_dev) {
  if (N % 256) throw std::runtime_error("mx_grouped_gemm_q_f32out: N % 256");
  MxGemvArgs a = gemm_args(nullptr, q, qs, K, tiles, w_tab, s_tab, nullptr, ldo, N, ntiles_dev, nullptr, nullptr,
                           nullptr, MxGlu{});
  a.out32 = out;
  launch_mx_gemm(a, ntiles, 0, st);
}

namespace {
int g_gemm_exact = -1;
}
// Exact dequantization is the default (the parity arithmetic); UH_GEMM_EXACT=0 in the environment selects the
// block-scaled MFMA, a speed mode whose sums are not exact (not a parity arithmetic).
bool mx_gemm_exact() {
  static const bool env = [] {
    const char* v = std::getenv("UH_GEMM_EXACT");
    return !(v && v[0] == '0');
  }();
  return g_gemm_exact < 0 ? env : g_gemm_exact > 0;
}
int mx_gemm_set_exact(int on) {
  const int prev = mx_gemm_exact() ? 1 : 0;
  g_gemm_exact = on ? 1 : 0;
  return prev;
}

void mx_grouped_gemm_x(const bf16* x, int ldx, const int32_t* x_rows, int K, const Exl3Tile* tiles, int ntiles,
                       const uint8_t* const* w_tab, const uint8_t* const* s_tab, bf16* out, int ldo, int N,
                       hipStream_t st, const int* ntiles_dev, const uint8_t* const* w_tab2,
                       const uint8_t* const* s_tab2, bf16* out2, const MxGlu& glu) {
  MxGemvArgs a = gemm_args(x, nullptr, nullptr, K, tiles, w_tab, s_tab, out, ldo, N, ntiles_dev, w_tab2, s_tab2, out2,
                           glu);
  a.x_rows = x_rows;
  a.ldx = ldx;
  launch_mx_gemm(a, ntiles, 2, st);
}

void mx_grouped_gemm_rows(const bf16* xa, const int32_t* x_rows, int K, const Exl3Tile* tiles, int ntiles,
                          const uint8_t* const* w_tab, const uint8_t* const* s_tab, bf16* out, int ldo, int N,
                          hipStream_t st, const int* ntiles_dev, const uint8_t* const* w_tab2,
                          const uint8_t* const* s_tab2, bf16* out2, const MxGlu& glu) {
  MxGemvArgs a = gemm_args(xa, nullptr, nullptr, K, tiles, w_tab, s_tab, out, ldo, N, ntiles_dev, w_tab2, s_tab2, out2,
                           glu);
  a.x_rows = x_rows;
  if (x_rows && (pipe_disabled() || K % GB_KS || N % 128))
    throw std::runtime_error("mx_grouped_gemm_rows: x_rows needs the pipelined kernel (K % 64, N % 128)");
  launch_mx_gemm(a, ntiles, 1, st);
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
