// Activation quantization and the fp8 e4m3 block-scaled dense GEMM/GEMV on gfx950, plus the reference-order
// a8w4 GEMM. Interfaces: include/unholy/kernels/ref.hpp, gemv.hpp, gemm_wmma.hpp.
//
// Dense fp8: C[M,N] = sum over 128-input blocks kb of raw_kb * scale(m, n, kb), raw_kb the exact fp8 dot over the
// block, fp32, bf16 out (ref_gemm.hip:130-137 with e8m0 scales; gemm_wmma.hip:89-100's fold for fp32 scales).
// On gfx950 raw_kb is four bf16 MFMAs (16x16x32) per 16 x 16 output tile on operands dequantized exactly in
// registers (the block-scaled f8f6f4 MFMA's internal sums are not fp32-accurate; see common.hpp).
#include <algorithm>
#include <type_traits>

#include "common.hpp"
#include "numerics.hpp"
#include "pipe.hpp"
#include "unholy/kernels/gemm_wmma.hpp"
#include "unholy/kernels/gemv.hpp"
#include "unholy/kernels/ref.hpp"
#include "fp8_internal.hpp"
#include "mx_internal.hpp"

namespace unholy::kernels {

using namespace uh;

namespace {

// act_quant per block of B values (B in {32, 64, 128}): a group of B/2 lanes, two values per lane.
// MODE 0: codes + e8m0 scale; 1: fake quant in place; 2: codes + fp32 scale (kernel.py scale_fmt=None).
template <int B, int MODE>
__global__ __launch_bounds__(256) void act_quant_kernel(const bf16* __restrict__ x, int ldx, uint8_t* __restrict__ q,
                                                        void* __restrict__ s, int rows, int cols) {
  constexpr int G = B / 2;
  const int nb = cols / B;
  const size_t gi = (blockIdx.x * size_t(blockDim.x) + threadIdx.x) / G;
  const int l = threadIdx.x % G;
  const bool valid = gi < size_t(rows) * nb;  // uniform per group of G lanes
  const int r = valid ? int(gi / nb) : 0, b = valid ? int(gi % nb) : 0;
  bf16* xr = const_cast<bf16*>(x) + size_t(r) * ldx + size_t(b) * B + 2 * l;
  float v0 = 0.0f, v1 = 0.0f;
  if (valid) {
    v0 = bf16_to_f32(xr[0]);
    v1 = bf16_to_f32(xr[1]);
  }
  const float am = group_max<G>(fmaxf(fabsf(v0), fabsf(v1)));
  if (!valid) return;
  uint8_t c0, c1;
  if constexpr (MODE == 2) {
    const float sc = fmaxf(am, 1e-4f) * (1.0f / 448.0f);
    c0 = fp8_code(v0, sc);
    c1 = fp8_code(v1, sc);
    if (l == 0) static_cast<float*>(s)[size_t(r) * nb + b] = sc;
  } else {
    const Fp8Block blk = fp8_block_scale(am);
    c0 = fp8_code(v0, blk);
    c1 = fp8_code(v1, blk);
    if constexpr (MODE == 1) {
      xr[0] = f32_to_bf16(e4m3_to_f32(c0) * blk.sc);
      xr[1] = f32_to_bf16(e4m3_to_f32(c1) * blk.sc);
      return;
    }
    if (l == 0) static_cast<uint8_t*>(s)[size_t(r) * nb + b] = blk.se;
  }
  *reinterpret_cast<uint16_t*>(q + size_t(r) * cols + size_t(b) * B + 2 * l) = uint16_t(c0 | uint32_t(c1) << 8);
}

// Block 128 with 8 values per thread: 16 consecutive threads per block (16-byte loads, 8-byte code stores), the amax a
// DPP row max. The item loop bound is uniform so every 16-lane group is whole. Needs ldx % 8 == 0.
template <int MODE>
__global__ __launch_bounds__(256) void act_quant8_kernel(const bf16* __restrict__ x, int ldx, uint8_t* __restrict__ q,
                                                         void* __restrict__ s, int rows, int cols) {
  const int nb = cols / 128;
  const size_t per_row = size_t(nb) * 16, items = size_t(rows) * per_row;
  for (size_t base = size_t(blockIdx.x) * 256; base < items; base += size_t(gridDim.x) * 256) {
    const size_t it = min(base + threadIdx.x, items - 1);
    const int r = int(it / per_row), rem = int(it % per_row), b = rem >> 4, l = rem & 15;
    bf16* xr = const_cast<bf16*>(x) + size_t(r) * ldx + size_t(b) * 128 + 8 * l;
    const uint4 raw = *reinterpret_cast<const uint4*>(xr);
    const uint32_t rw[4] = {raw.x, raw.y, raw.z, raw.w};
    float v[8], am = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(rw[i] << 16);
      v[2 * i + 1] = __uint_as_float(rw[i] & 0xffff0000u);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) am = fmaxf(am, fabsf(v[i]));
    am = row16_max(am);
    if (base + threadIdx.x >= items) continue;
    uint32_t c[2];
    if constexpr (MODE == 2) {
      const float sc = fmaxf(am, 1e-4f) * (1.0f / 448.0f);
      fp8_codes8(v, sc, c[0], c[1]);
      if (l == 0) static_cast<float*>(s)[size_t(r) * nb + b] = sc;
    } else {
      const Fp8Block blk = fp8_block_scale(am);
      fp8_codes8(v, blk, c[0], c[1]);
      if constexpr (MODE == 1) {  // the fake-quantized values: the codes decoded back (exact)
        *reinterpret_cast<uint4*>(xr) = __builtin_bit_cast(uint4, fp8x8_to_bf16(c[0], c[1], blk.sc));
        continue;
      }
      if (l == 0) static_cast<uint8_t*>(s)[size_t(r) * nb + b] = blk.se;
    }
    *reinterpret_cast<uint2*>(q + size_t(r) * cols + size_t(b) * 128 + 8 * l) = make_uint2(c[0], c[1]);
  }
}

template <int MODE>
void launch_act_quant(const bf16* x, int ldx, uint8_t* q, void* s, int rows, int cols, int block, hipStream_t st) {
  if (rows <= 0) return;
  if (block != 32 && block != 64 && block != 128) throw std::runtime_error("act_quant: block in {32, 64, 128}");
  if (cols % block) throw std::runtime_error("act_quant: cols % block");
  if (block == 128 && ldx % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 && (MODE == 1 || cols % 8 == 0)) {
    const unsigned grid = unsigned(std::min<size_t>(cdiv(size_t(rows) * (cols / 8), 256), 8192));
    act_quant8_kernel<MODE><<<grid, 256, 0, st>>>(x, ldx, q, s, rows, cols);
    UH_CHECK_LAUNCH();
    return;
  }
  const size_t threads = size_t(rows) * (cols / block) * (block / 2);
  const unsigned grid = cdiv(threads, 256);
  if (block == 32) act_quant_kernel<32, MODE><<<grid, 256, 0, st>>>(x, ldx, q, s, rows, cols);
  else if (block == 64) act_quant_kernel<64, MODE><<<grid, 256, 0, st>>>(x, ldx, q, s, rows, cols);
  else act_quant_kernel<128, MODE><<<grid, 256, 0, st>>>(x, ldx, q, s, rows, cols);
  UH_CHECK_LAUNCH();
}

// ---- reference-order a8w4 GEMM ----------------------------------------------------------------------------------
// A thread per output: per 32-block the exact partial sum in k order, scaled by sa[m][k/128] * sw[n][k/32] and
// added in block order -- the operation order of the reference's gemm_a8w4 (ref_gemm.hip:26-58, G = 32), so the
// fp32 results are the reference's bit for bit. Not a fast path: a pinned twin of the MFMA kernels.
template <bool TILED>
__global__ __launch_bounds__(256) void gemm_a8w4_ref_kernel(const uint8_t* a, const uint8_t* sa, const uint8_t* w,
                                                            const uint8_t* sw, bf16* c, int ldc, int M, int N, int K) {
  const int n = blockIdx.x * 256 + threadIdx.x, m = blockIdx.y;
  if (n >= N) return;
  float acc = 0.0f;
  for (int kb = 0; kb < K / 32; ++kb) {
    float part = 0.0f;
    for (int k = kb * 32; k < kb * 32 + 32; ++k) {
      uint8_t byte;
      if constexpr (TILED) byte = w[(size_t(k / 64) * (N / 16) + n / 16) * 512 + (n % 16) * 32 + (k % 64) / 2];
      else byte = w[size_t(n) * (K / 2) + k / 2];
      part = fmaf(e4m3_to_f32(a[size_t(m) * K + k]), e2m1_to_f32((k & 1) ? (byte >> 4) : (byte & 0xf)), part);
    }
    uint8_t sb;
    if constexpr (TILED) sb = sw[(size_t(kb / 2) * (N / 16) + n / 16) * 32 + (n % 16) * 2 + kb % 2];
    else sb = sw[size_t(n) * (K / 32) + kb];
    acc += part * (e8m0_to_f32(sa[size_t(m) * (K / 128) + kb / 4]) * e8m0_to_f32(sb));
  }
  c[size_t(m) * ldc + n] = f32_to_bf16(acc);
}

// ---- fp8 dense, skinny (rows in groups of <= 16 staged in LDS) -------------------------------------------------------
// A workgroup = 4 waves x DN_TN 16-column tiles. Per 128-input step lane l takes 32 code bytes of weight row
// n0 + l % 16 at inputs 32 (l / 16) .. + 31 (four lanes cover one row's 128 contiguous bytes), dequantizes them and
// the matching activation inputs exactly to bf16 and issues four bf16 MFMAs per column tile. e8m0 scales are
// folded into the conversions (exact) and the MFMA accumulates across blocks; with fp32 scales each 128-block's
// MFMA chain starts from zero and is folded as acc += raw * (sa * sw), the reference's order of scaling.
constexpr int DN_NT = 256, DN_WAVES = 4, DN_TN = 2, DN_PAD = 16, DN_MAXROWS = 16;

template <bool F32S>
__global__ __launch_bounds__(DN_NT) void fp8_skinny_kernel(Fp8GemmArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int K = a.K, N = a.N, KS = K / 128, ldA = K + DN_PAD, ntn = (N + 15) / 16;
  uint8_t* sA = smem;
  float* sSf = reinterpret_cast<float*>(smem + size_t(a.rows_cap) * ldA);
  uint8_t* sSb = smem + size_t(a.rows_cap) * ldA;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, nl = lane & 15, g = lane >> 4;
  int nt[DN_TN];
#pragma unroll
  for (int j = 0; j < DN_TN; ++j) nt[j] = blockIdx.x * (DN_WAVES * DN_TN) + wave * DN_TN + j;
  const int rg = blockIdx.y * a.rows_cap, M = min(a.rows_cap, a.M - rg);
  for (int i = tid; i < M * (K / 16); i += DN_NT) {
    const int m = i / (K / 16), c = (i % (K / 16)) * 16;
    *reinterpret_cast<uint4*>(sA + m * ldA + c) = *reinterpret_cast<const uint4*>(a.a + size_t(rg + m) * K + c);
  }
  for (int i = tid; i < M * KS; i += DN_NT) {
    if constexpr (F32S) sSf[i] = a.sa32[size_t(rg) * KS + i];
    else sSb[i] = a.sa8[size_t(rg) * KS + i];
  }
  __syncthreads();
  const bool arow = nl < M;
  const uint8_t* ap = sA + nl * ldA + g * 32;
  v4f acc[DN_TN];
#pragma unroll
  for (int j = 0; j < DN_TN; ++j) acc[j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  // Weight row of this lane in each column tile (rows past N read row N - 1 and are not stored).
  const uint8_t* wrow[DN_TN];
#pragma unroll
  for (int j = 0; j < DN_TN; ++j) wrow[j] = a.w + size_t(min(nt[j] * 16 + nl, N - 1)) * K + g * 32;
#pragma unroll 2
  for (int s = 0; s < KS; ++s) {
    v4i b[DN_TN][2];
#pragma unroll
    for (int j = 0; j < DN_TN; ++j)
      if (nt[j] < ntn) {
        b[j][0] = *reinterpret_cast<gptr<v4i>>(as_global(wrow[j] + s * 128));
        b[j][1] = *reinterpret_cast<gptr<v4i>>(as_global(wrow[j] + s * 128 + 16));
      }
    // Activation inputs 32g .. 32g + 31 of row nl (scale folded in for e8m0, 1.0 for fp32 scales).
    bf16x8 af[4];
    if (arow) {
      const v4i lo = *reinterpret_cast<const v4i*>(ap + s * 128), hi = *reinterpret_cast<const v4i*>(ap + s * 128 + 16);
      const float sc = F32S ? 1.0f : e8m0_to_f32(sSb[nl * KS + s]);
      af[0] = fp8x8_to_bf16(lo[0], lo[1], sc);
      af[1] = fp8x8_to_bf16(lo[2], lo[3], sc);
      af[2] = fp8x8_to_bf16(hi[0], hi[1], sc);
      af[3] = fp8x8_to_bf16(hi[2], hi[3], sc);
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t) af[t] = bf16x8{};
    }
    if constexpr (F32S) {
      float sa_i[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) sa_i[i] = (4 * g + i) < M ? sSf[(4 * g + i) * KS + s] : 0.0f;
#pragma unroll
      for (int j = 0; j < DN_TN; ++j)
        if (nt[j] < ntn) {
          v4f raw = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int t = 0; t < 4; ++t)
            raw = mfma_bf16(af[t], fp8x8_to_bf16(uint32_t(b[j][t / 2][2 * (t % 2)]), uint32_t(b[j][t / 2][2 * (t % 2) + 1]), 1.0f), raw);
          const float swv = a.sw32[size_t(min(nt[j] * 16 + nl, N - 1) / 128) * KS + s];
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[j][i] += raw[i] * (sa_i[i] * swv);
        }
    } else {
#pragma unroll
      for (int j = 0; j < DN_TN; ++j)
        if (nt[j] < ntn) {
          const float sc = e8m0_to_f32(a.sw8[size_t(min(nt[j] * 16 + nl, N - 1) / 128) * KS + s]);
#pragma unroll
          for (int t = 0; t < 4; ++t)
            acc[j] = mfma_bf16(af[t], fp8x8_to_bf16(uint32_t(b[j][t / 2][2 * (t % 2)]), uint32_t(b[j][t / 2][2 * (t % 2) + 1]), sc), acc[j]);
        }
    }
  }
#pragma unroll
  for (int j = 0; j < DN_TN; ++j) {
    const int n = nt[j] * 16 + nl;
    if (nt[j] >= ntn || n >= N) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * g + i;
      if (r < M) a.c[size_t(rg + r) * a.ldc + n] = f32_to_bf16(acc[j][i]);
    }
  }
}

// ---- fp8 dense, small M (<= 64 rows): bandwidth-shaped --------------------------------------------------------------
// One workgroup per 16-column tile; its 8 waves split K (wave w takes 128-blocks w * per .. + per - 1), so the grid
// covers every CU and each CU keeps 8 waves x 64 lanes x 128 B of weights in flight (four 128-blocks per wave are
// loaded before any is used). Lane (nl, g) reads 32 weight bytes of column n0 + nl at inputs 32g .. + 31 of a block
// and the same inputs of activation row nl (row tile mt: rows 16 mt + nl) from global memory (A is small and
// cache-resident), dequantizes both exactly to bf16 (e8m0 scales folded in) and issues 16x16x32 bf16 MFMAs. With fp32
// scales each block's MFMA chain starts from zero and is folded as acc += raw * (sa * sw). The 8 partial tiles are
// summed in wave order through LDS.
constexpr int FV_WAVES = 8, FV_CHUNK = 4;

// XQ: A arrives as bf16 rows (a.xa). The workgroup first quantizes its M rows into LDS as act_quant_fp8_f32s does
// (s = max(amax, 1e-4) * fp32(1/448), codes e4m3(x / s); 8 values per thread, a block's amax a DPP row max over its
// 16 threads; all waves, before the K loop, so that a wave with no K blocks still meets the barrier), then reads
// codes and scales from LDS. Same codes and
// scales as the separate quantization, so the same results bit for bit, one launch fewer.
template <bool F32S, int MT, bool XQ = false>
__global__ __launch_bounds__(64 * FV_WAVES) void fp8_gemv_kernel(Fp8GemmArgs a, Fp8Parts pp) {
  static_assert(!XQ || (F32S && MT == 1), "the fused quantization: fp32 scales, one row tile");
  __shared__ v4f red[FV_WAVES][MT][64];
  extern __shared__ __align__(16) uint8_t xq_lds[];  // XQ: codes [M][K], then fp32 scales [M][K / 128]
  int tile = blockIdx.x;
  if (pp.n) {  // column ranges: this workgroup's range (uniform)
    int p = 0;
    while (p + 1 < pp.n && tile >= pp.t0[p + 1]) ++p;
    tile -= pp.t0[p];
    a.w = pp.w[p];
    a.sw8 = pp.sw[p];
    a.c = pp.c[p];
    a.ldc = pp.ldc[p];
    a.N = pp.N[p];
  }
  const int K = a.K, KS = K / 128, N = a.N, M = a.M;
  const int tid = threadIdx.x, lane = tid & 63, nl = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n0 = tile * 16, n = min(n0 + nl, N - 1), nb = n0 / 128;  // a 16-column tile lies in one 128-block
  const int per = (KS + FV_WAVES - 1) / FV_WAVES, b0 = min(KS, wave * per), b1 = min(KS, b0 + per);
  const uint8_t* wrow = a.w + size_t(n) * K + g * 32;
  v4f acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  const int mlive = (M + 15) / 16;  // row tiles with rows (uniform)
  // The chunk's weights and their scales (every load issued before the first use; steps past the range clamped).
  v4i b[FV_CHUNK][2];
  float swv[FV_CHUNK];
  const auto load_weights = [&](int kc) {
#pragma unroll
    for (int u = 0; u < FV_CHUNK; ++u) {
      const int kb = min(kc + u, b1 - 1);
      b[u][0] = *reinterpret_cast<gptr<v4i>>(as_global(wrow + kb * 128));
      b[u][1] = *reinterpret_cast<gptr<v4i>>(as_global(wrow + kb * 128 + 16));
      swv[u] = F32S ? a.sw32[size_t(nb) * KS + kb] : e8m0_to_f32(a.sw8[size_t(nb) * KS + kb]);
    }
  };
  if constexpr (XQ) {  // every wave: quantize the M rows into LDS before any wave reads them
    const int nbk = KS * 16, items = M * nbk;  // 8 values per item
    float* const sl = reinterpret_cast<float*>(xq_lds + size_t(M) * K);
    const auto load_item = [&](int base) {
      const int it = min(base + tid, items - 1), r = it / nbk, rem = it % nbk, bk = rem >> 4, l = rem & 15;
      return *reinterpret_cast<const uint4*>(a.xa + size_t(r) * a.ldx + bk * 128 + 8 * l);
    };
    const auto quant_item = [&](int base, const uint4 raw) {
      const int it = min(base + tid, items - 1), r = it / nbk, rem = it % nbk, bk = rem >> 4, l = rem & 15;
      const uint32_t rw[4] = {raw.x, raw.y, raw.z, raw.w};
      float v[8], am = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float(rw[i] << 16);
        v[2 * i + 1] = __uint_as_float(rw[i] & 0xffff0000u);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) am = fmaxf(am, fabsf(v[i]));
      am = row16_max(am);
      if (base + tid >= items) return;
      const float sc = fmaxf(am, 1e-4f) * (1.0f / 448.0f);
      uint32_t c0, c1;
      fp8_codes8(v, sc, c0, c1);
      *reinterpret_cast<uint2*>(xq_lds + size_t(r) * K + bk * 128 + 8 * l) = make_uint2(c0, c1);
      if (l == 0) sl[r * KS + bk] = sc;
    };
    // The first pass's row loads, then the first chunk's weights, then the quantization: it waits for the row loads
    // only, and the weights' latency runs under it.
    // (A wave with no K blocks loads block KS - 1 and never uses it: an unconditional load keeps the wait exact.)
    const uint4 raw0 = load_item(0);
    load_weights(b0);
    quant_item(0, raw0);
    for (int base = 64 * FV_WAVES; base < items; base += 64 * FV_WAVES)  // uniform bound: 16-thread groups stay whole
      quant_item(base, load_item(base));
    __syncthreads();
  }
  for (int kc = b0; kc < b1; kc += FV_CHUNK) {
    // Every load of the chunk is issued before the first use, unconditionally (steps past the range and rows past M
    // are clamped, their products discarded): the weights, the activation rows and the scales, so the chunk waits
    // for one memory latency, not one per step.
    v4i aq[FV_CHUNK][MT][2];
    float sav[FV_CHUNK][MT];
    constexpr bool kRowScales = F32S && MT == 1;  // the fp32 row scales of C's rows too (registers permitting)
    float sa32v[FV_CHUNK][4];
    if (!XQ || kc != b0) load_weights(kc);
#pragma unroll
    for (int u = 0; u < FV_CHUNK; ++u) {
      const int kb = min(kc + u, b1 - 1);
      if constexpr (XQ) {
        sav[u][0] = 1.0f;
      } else {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int r = min(mt * 16 + nl, M - 1);
          const uint8_t* ap = a.a + size_t(r) * K + kb * 128 + g * 32;
          aq[u][mt][0] = *reinterpret_cast<gptr<v4i>>(as_global(ap));
          aq[u][mt][1] = *reinterpret_cast<gptr<v4i>>(as_global(ap + 16));
          sav[u][mt] = F32S ? 1.0f : e8m0_to_f32(a.sa8[size_t(r) * KS + kb]);
        }
        if constexpr (kRowScales)
#pragma unroll
          for (int i = 0; i < 4; ++i) sa32v[u][i] = a.sa32[size_t(min(4 * g + i, M - 1)) * KS + kb];
      }
    }
    if constexpr (XQ) {  // codes and C rows' scales from the LDS copy
      const float* const sl = reinterpret_cast<const float*>(xq_lds + size_t(M) * K);
#pragma unroll
      for (int u = 0; u < FV_CHUNK; ++u) {
        const int kb = min(kc + u, b1 - 1);
        const uint8_t* ap = xq_lds + size_t(min(nl, M - 1)) * K + kb * 128 + g * 32;
        aq[u][0][0] = *reinterpret_cast<const v4i*>(ap);
        aq[u][0][1] = *reinterpret_cast<const v4i*>(ap + 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) sa32v[u][i] = sl[min(4 * g + i, M - 1) * KS + kb];
      }
    }
#pragma unroll
    for (int u = 0; u < FV_CHUNK; ++u) {
      const int kb = kc + u;
      if (kb >= b1) break;
      bf16x8 bf[4];
#pragma unroll
      for (int t = 0; t < 4; ++t)
        bf[t] = fp8x8_to_bf16(uint32_t(b[u][t / 2][2 * (t % 2)]), uint32_t(b[u][t / 2][2 * (t % 2) + 1]),
                              F32S ? 1.0f : swv[u]);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if (mt >= mlive) break;
        bf16x8 af[4];
        if (mt * 16 + nl < M) {
          const v4i lo = aq[u][mt][0], hi = aq[u][mt][1];
          af[0] = fp8x8_to_bf16(lo[0], lo[1], sav[u][mt]);
          af[1] = fp8x8_to_bf16(lo[2], lo[3], sav[u][mt]);
          af[2] = fp8x8_to_bf16(hi[0], hi[1], sav[u][mt]);
          af[3] = fp8x8_to_bf16(hi[2], hi[3], sav[u][mt]);
        } else {
#pragma unroll
          for (int t = 0; t < 4; ++t) af[t] = bf16x8{};
        }
        if constexpr (F32S) {
          v4f raw = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int t = 0; t < 4; ++t) raw = mfma_bf16(af[t], bf[t], raw);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int rr = mt * 16 + 4 * g + i;  // C row of value i
            const float sa = rr >= M ? 0.0f : kRowScales ? sa32v[u][i] : a.sa32[size_t(rr) * KS + kb];
            acc[mt][i] += raw[i] * (sa * swv[u]);
          }
        } else {
#pragma unroll
          for (int t = 0; t < 4; ++t) acc[mt] = mfma_bf16(af[t], bf[t], acc[mt]);
        }
      }
    }
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) red[wave][mt][lane] = acc[mt];
  __syncthreads();
  // Wave w < MT stores row tile w: the sum of the 8 partials in wave order.
  if (wave < MT && wave * 16 < M) {
    v4f s = red[0][wave][lane];
#pragma unroll
    for (int w = 1; w < FV_WAVES; ++w) s += red[w][wave][lane];
    if (n0 + nl < N)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = wave * 16 + 4 * g + i;
        if (r < M) a.c[size_t(r) * a.ldc + n0 + nl] = f32_to_bf16(s[i]);
      }
  }
}

void launch_fp8_gemv_xq(const Fp8GemmArgs& a, hipStream_t st) {
  const size_t lds = size_t(a.M) * a.K + size_t(a.M) * (a.K / 128) * 4;
  auto* kern = &fp8_gemv_kernel<true, 1, true>;
  UH_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                               int(lds)));
  kern<<<dim3(unsigned(cdiv(size_t(a.N), 16))), 64 * FV_WAVES, lds, st>>>(a, Fp8Parts{});
  UH_CHECK_LAUNCH();
}

template <bool F32S>
void launch_fp8_gemv_t(const Fp8GemmArgs& a, hipStream_t st, const Fp8Parts& pp) {
  const dim3 grid(unsigned(pp.n ? pp.t0[pp.n] : cdiv(size_t(a.N), 16)));
  if (a.M <= 16) fp8_gemv_kernel<F32S, 1><<<grid, 64 * FV_WAVES, 0, st>>>(a, pp);
  else fp8_gemv_kernel<F32S, 4><<<grid, 64 * FV_WAVES, 0, st>>>(a, pp);
  UH_CHECK_LAUNCH();
}


// ---- fp8 dense, 16 < M <= 256 with fp32 scales: row tiles ------------------------------------------------------------
// A workgroup per 32 columns x 32 rows over the whole of K (<= 8,192), bf16 C written directly, one launch:
// - 16 waves = 16 K parts of one 32 x 32 output tile (bf16 MFMA 32x32x16); part p takes block p of every 2,048-input
//   chunk;
// - CH = 1: each wave loads the activation codes of its own K part (32 rows x 128 codes a chunk, four 1 KB loads)
//   into its own 2-slot LDS ring by direct global -> LDS loads, and its rows' fp32 scales into registers (lane r
//   holds row r's; a lane-crossbar read hands each accumulator row its scale). No wave waits for another before the
//   final reduction, so a wave computes its chunks as soon as its own loads land while the others still stream;
//   piece q (16 bytes) of row r sits at q ^ ((r >> 1) & 7), so a 16-lane pass of 16-byte reads covers the 64 banks
//   once. The waves of a 32-row tile share nothing but the reduction;
// - CH = 2 (the two column halves of a K part read the same activations): the tile's activation codes go through a
//   2-slot LDS ring of chunks (32 rows x 1,024 codes, 32 KB) by direct global -> LDS loads, filled by all 16 waves and
//   read after a barrier; piece p (16 bytes) of row r sits at p ^ (r & 15), so a 16-lane pass of 16-byte reads
//   covers the 64 banks once; the fp32 row scales of the tile are staged beside them;
// - a wave's weights for all (<= 4) chunks are loaded into registers up front, interleaved with the first two
//   activation chunks (issue order: scales, W0 A0 W1 A1 W2 W3, then A(c + 2) once chunk c is done); loads retire in
//   order and each chunk waits for exactly the loads before its own. Weight load x (0..3) of a block: lane l reads
//   16 bytes of column 16 (x >> 1) + l % 16 at byte 64 (x & 1) + 16 (l >> 4) (64 contiguous bytes of each of 16
//   rows); one lane-row swap per dword pair then leaves lane l with column l % 32, load x holding piece
//   2 h + (x >> 1) + 4 (x & 1) of the block, and the activation reads take the same pieces;
// - per block: the raw chain of 8 MFMAs on exactly converted codes, folded as acc += raw * (sa * sw) (the reference's
//   fp32-scale order); the 16 parts are added in LDS in part order, wave p adding accumulator element p;
// - work item wi = column block x row tiles + row tile; XCD x takes the x-th eighth of the items, so the row tiles of
//   a column block share one L2.
// Against the one-tile GEMV (every 16-column workgroup reading all M rows from L2): the rows leave L2 once per 32
// columns. A K split over workgroups (fp32 partial tiles in a workspace, added in slice order by a second launch) ran
// 17.9 us per step at 64 x 4096 x 4096 against 14.0 here: the second launch and the partial round trip cost more
// than the split gains.
// Up to FR_MAXM rows (8 row tiles): at 4096 x 4096 the row tiles ran 22-43 us per step for 65 <= M <= 256 against
// 47-53 us for the 128 x 128 tiled GEMM (too few workgroups there), which wins from M = 384 on (53 against 62 us).
constexpr int FR_MAXCH = 4, FR_MAXM = 256;

// CH column halves of 32 (workgroup width 32 CH); KP = 16 / CH K parts; chunks of KR = 128 KP inputs; NA direct loads
// per wave per chunk (32 rows x KR codes in 1 KB loads over 16 waves). CH = 2 halves the workgroups of a wide, short
// matrix (N / 64 column blocks), each wave then adding two accumulator elements in the reduction.
template <int CH>
struct Fp8Rows {
  static constexpr int KP = 16 / CH, KR = 128 * KP, SLOT = 32 * KR, NA = SLOT / 1024 / 16, W = 32 * CH;
  static constexpr int LS = CH == 2 ? 18 : 17;  // reduction lane stride (floats)
  // CH = 1: each wave's own 2-slot ring of its K part (32 rows x 128 codes, 4 KB a slot); CH = 2: the shared ring
  // of chunks and the tile's row scales.
  static size_t lds(int K) {
    const size_t ring = CH == 1 ? size_t(16) * 2 * 4096 : 2 * size_t(SLOT) + size_t(32) * (K / 128) * 4;
    return std::max(ring, size_t(16) * 64 * LS * 4);
  }
};

// NCH = the chunk count, ceil((K / 128) / KP) (1..FR_MAXCH): a template parameter, so that the issue order and every
// counted wait are fixed at compile time and no branch depends on how many loads are outstanding.
template <int CH, int NCH>
__global__ __launch_bounds__(1024) void fp8_rows_kernel(Fp8GemmArgs p) {
  using namespace pipe;
  using T = Fp8Rows<CH>;
  constexpr int KP = T::KP, KR = T::KR, SLOT = T::SLOT, NA = T::NA;
  extern __shared__ __align__(16) uint8_t smem[];
  static_assert(NCH >= 1 && NCH <= FR_MAXCH);
  static_assert(CH == 2 || NA == 4, "CH = 1: four 1 KB activation loads per wave and chunk");
  const int M = p.M, N = p.N, K = p.K, KS = K / 128;  // the host launches NCH = ceil(KS / KP)
  const int nw = gridDim.x, lin = blockIdx.x;
  const int wi = nw % 8 ? lin : (lin & 7) * (nw >> 3) + (lin >> 3);
  const int RT = (M + 31) / 32, rt = wi % RT, bx = wi / RT, row0 = rt * 32;
  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), chh = wave % CH, kh = wave / CH;  // column half, K part
  const int col0 = bx * T::W, n = col0 + chh * 32 + l32;
  const uint8_t* wld = p.w + size_t(col0 + chh * 32 + (lane & 15)) * K + (lane >> 4) * 16;
  const float* swrow = p.sw32 + size_t((col0 + chh * 32) / 128) * KS;  // 32 columns lie in one 128-row block
  const uint32_t lds0 = lds_addr(smem);
  // The activation loads. CH = 1: load i of the wave covers rows 8i .. 8i + 7 of its 4 KB slot, lane j row
  // 8i + j / 8 at piece (j % 8) ^ swz(row) of the K part. CH = 2: load i covers 1 KB of the shared chunk slot.
  uint32_t rowoff[NA];
  int pin[NA];
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    if constexpr (CH == 1) {
      const int r = 8 * i + (lane >> 3);
      rowoff[i] = uint32_t(min(row0 + r, M - 1)) * uint32_t(K);
      pin[i] = 16 * ((lane & 7) ^ ((r >> 1) & 7));
    } else {
      const int slot = (wave * NA + i) * 64 + lane, r = slot / (KR / 16);
      rowoff[i] = uint32_t(min(row0 + r, M - 1)) * uint32_t(K);
      pin[i] = ((slot % (KR / 16)) ^ (r & 15)) * 16;
    }
  }
  const auto issue_a = [&](int ch) {
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      if constexpr (CH == 1)
        dma16(p.a, rowoff[i] + uint32_t(min(ch * KP + kh, KS - 1)) * 128u + uint32_t(pin[i]),
              lds0 + uint32_t((wave * 2 + (ch & 1)) * 4096 + i * 1024));
      else
        dma16(p.a, rowoff[i] + uint32_t(min(ch * KR + pin[i], K - 16)),
              lds0 + uint32_t((ch & 1) * SLOT + (wave * NA + i) * 1024));
    }
  };
  v4i b[NCH][4];
  const auto load_w = [&](int u) {
    const uint8_t* q = wld + min(u * KP + kh, KS - 1) * 128;
#pragma unroll
    for (int x = 0; x < 4; ++x) b[u][x] = vload16(q + (x >> 1) * 16 * K + (x & 1) * 64);
  };
  // Issue order: the scales (lane u < nch: the wave's weight scale of chunk u; CH = 1: lane r's row scale of each
  // chunk's block; CH = 2: thread t's row scales t, t + 1024 of the tile), W0 A0 W1 A1 W2 W3, then A(c + 2).
  uint32_t swv = vload_u32(swrow + min(min(lane, FR_MAXCH - 1) * KP + kh, KS - 1));
  constexpr int NSA = CH == 1 ? NCH : 2;
  uint32_t sav[NSA];
#pragma unroll
  for (int j = 0; j < NSA; ++j) {
    if constexpr (CH == 1) {
      sav[j] = vload_u32(p.sa32 + size_t(min(row0 + l32, M - 1)) * KS + min(j * KP + kh, KS - 1));
    } else {
      const int e = min(tid + 1024 * j, 32 * KS - 1);
      sav[j] = vload_u32(p.sa32 + size_t(min(row0 + e / KS, M - 1)) * KS + e % KS);
    }
  }
  float* const ssa = reinterpret_cast<float*>(smem + 2 * SLOT);  // CH = 2: row scales [32][KS]
  load_w(0);
  issue_a(0);
  if constexpr (NCH > 1) {
    load_w(1);
    issue_a(1);
  }
  if constexpr (NCH > 2) load_w(2);
  if constexpr (NCH > 3) load_w(3);
  const int r = l32;
  v16f_t acc = v16f_t{};
  const auto chunk = [&](auto ich) {
    constexpr int ch = decltype(ich)::value;
    // Chunk ch, its weights and the scales have landed when only the loads issued after A(ch) are pending (4 per
    // weight group, NA per activation group): ch = 0: W1 A1 W2 W3; ch = 1: W2 W3 A2; ch = 2: A3; each where it
    // exists.
    constexpr int later = ch == 0   ? 4 * ((1 < NCH) + (2 < NCH) + (3 < NCH)) + NA * (1 < NCH)
                          : ch == 1 ? 4 * ((2 < NCH) + (3 < NCH)) + NA * (2 < NCH)
                          : ch == 2 ? NA * (3 < NCH)
                                    : 0;
    wait_vm<later>();
    vlanded(b[ch]);
    if (ch == 0) {
      vlanded(swv);
#pragma unroll
      for (int j = 0; j < NSA; ++j) vlanded(sav[j]);
      if constexpr (CH == 2)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          if (tid + 1024 * j < 32 * KS) ssa[tid + 1024 * j] = __uint_as_float(sav[j]);
    }
    if constexpr (CH == 1) asm volatile("" ::: "memory");  // the wave's own activation pieces have landed in LDS
    else __syncthreads();                                    // every wave's part of chunk ch (and the row scales)
    const int kb = ch * KP + kh;
    if (kb < KS) {
      const uint8_t* sl = CH == 1 ? smem + (wave * 2 + (ch & 1)) * 4096 : smem + (ch & 1) * SLOT;
      const float sw = __uint_as_float(uint32_t(__builtin_amdgcn_readlane(int(swv), ch)));
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          // Lanes 16-31 (48-63) of load x trade with lanes 0-15 (32-47) of load x + 2.
          const auto t = __builtin_amdgcn_permlane16_swap(uint32_t(b[ch][x][d]), uint32_t(b[ch][x + 2][d]), false,
                                                          false);
          b[ch][x][d] = int(t[0]);
          b[ch][x + 2][d] = int(t[1]);
        }
      v16f_t raw = v16f_t{};
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        const int q = 2 * h + (x >> 1) + 4 * (x & 1);  // the piece of the block this load holds
        const v4i av = CH == 1 ? *reinterpret_cast<const v4i*>(sl + r * 128 + (q ^ ((r >> 1) & 7)) * 16)
                               : *reinterpret_cast<const v4i*>(sl + r * KR + ((kh * 8 + q) ^ (r & 15)) * 16);
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const bf16x8 af = fp8x8_to_bf16(uint32_t(av[2 * e]), uint32_t(av[2 * e + 1]), 1.0f);
          const bf16x8 bf = fp8x8_to_bf16(uint32_t(b[ch][x][2 * e]), uint32_t(b[ch][x][2 * e + 1]), 1.0f);
          raw = mfma32_bf16(af, bf, raw);
        }
      }
      // Element i of lane (l32, h) is row 8 (i / 4) + 4 h + i % 4 of the tile.
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = 8 * (i / 4) + 4 * h + (i % 4);
        float sa;
        if constexpr (CH == 1)
          sa = __uint_as_float(uint32_t(__builtin_amdgcn_ds_bpermute(row * 4, int(sav[ch]))));
        else
          sa = ssa[row * KS + kb];
        acc[i] += raw[i] * (sa * sw);
      }
    }
    if constexpr (ch + 2 < NCH) {
      if constexpr (CH == 2) __syncthreads();  // every wave is done with slot ch & 1
      issue_a(ch + 2);  // CH = 1: the wave's own slot, whose reads above have returned
    }
  };
  chunk(std::integral_constant<int, 0>{});
  if constexpr (NCH > 1) chunk(std::integral_constant<int, 1>{});
  if constexpr (NCH > 2) chunk(std::integral_constant<int, 2>{});
  if constexpr (NCH > 3) chunk(std::integral_constant<int, 3>{});
  // The KP parts added in part order through LDS: wave (chh, kh) adds elements CH kh .. CH kh + CH - 1 of its column
  // half's lanes (lane stride 17 floats for 4-byte reads, 18 for 8-byte ones: a half-wave's reads cover the 64 banks
  // once).
  __syncthreads();
  float* red = reinterpret_cast<float*>(smem);
  float* mine = red + ((kh * CH + chh) * 64 + lane) * T::LS;
  if constexpr (CH == 2) {
#pragma unroll
    for (int i = 0; i < 16; i += 2) *reinterpret_cast<float2*>(mine + i) = make_float2(acc[i], acc[i + 1]);
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) mine[i] = acc[i];
  }
  __syncthreads();
  float sum[CH];
#pragma unroll
  for (int e = 0; e < CH; ++e) sum[e] = red[(chh * 64 + lane) * T::LS + CH * kh + e];
#pragma unroll
  for (int q = 1; q < KP; ++q)
#pragma unroll
    for (int e = 0; e < CH; ++e) sum[e] += red[((q * CH + chh) * 64 + lane) * T::LS + CH * kh + e];
  // Element i of lane (l32, h) is row 8 (i / 4) + 4 h + i % 4 of the tile.
#pragma unroll
  for (int e = 0; e < CH; ++e) {
    const int i = CH * kh + e, row = row0 + 8 * (i / 4) + 4 * h + (i % 4);
    if (row < M) p.c[size_t(row) * p.ldc + n] = f32_to_bf16(sum[e]);
  }
}
}  // namespace

// The wide form (CH = 2, K <= 4096) where its rounds of workgroups (256 CUs, one workgroup each) cost less: a wide
// workgroup runs ~1.7x as long as a narrow one (~1.25x at K <= 1024, where half the narrow form's K parts idle).
// Measured (us per call, wide / narrow): 32768 x 1024 M = 64 26.8 / 43.1, 8192 x 1024 M = 64 7.4 / 11.6, 4096 x 4096
// M = 128 17.2 / 20.3, 129280 x 4096 M = 32 150 / 174; M = 64 at 4096 x 4096 (128 wide workgroups) 16.9 / 11.8, and
// M = 160 (320 against 640 workgroups) 34.6 / 31.8 per step.
static bool fp8_rows_wide(const Fp8GemmArgs& a) {
  if (a.N % 64 || a.K > FR_MAXCH * Fp8Rows<2>::KR) return false;
  const size_t rt = size_t(a.M + 31) / 32, nn = size_t(a.N / 32) * rt, nw = size_t(a.N / 64) * rt;
  const double f = a.K <= 1024 ? 1.25 : 1.7;
  return double((nw + 255) / 256) * f < double((nn + 255) / 256);
}
bool fp8_rows_fits(const Fp8GemmArgs& a) {
  return a.sa32 && a.sw32 && a.M > 16 && a.M <= FR_MAXM && a.N % 32 == 0 && a.K % 128 == 0 && a.K >= 128 &&
         a.K <= FR_MAXCH * Fp8Rows<1>::KR && size_t(a.M) * a.K < (size_t(1) << 32);
}
template <int CH>
static void launch_fp8_rows_t(const Fp8GemmArgs& a, hipStream_t st) {
  const size_t lds = Fp8Rows<CH>::lds(a.K);
  const int nch = (a.K / 128 + Fp8Rows<CH>::KP - 1) / Fp8Rows<CH>::KP;  // 1..FR_MAXCH (fp8_rows_fits)
  auto* kern = nch == 1   ? &fp8_rows_kernel<CH, 1>
               : nch == 2 ? &fp8_rows_kernel<CH, 2>
               : nch == 3 ? &fp8_rows_kernel<CH, 3>
                          : &fp8_rows_kernel<CH, 4>;
  UH_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                               int(lds)));
  kern<<<dim3(unsigned(a.N / Fp8Rows<CH>::W * ((a.M + 31) / 32))), 1024, lds, st>>>(a);
  UH_CHECK_LAUNCH();
}
void launch_fp8_rows(const Fp8GemmArgs& a, hipStream_t st) {
  if (!fp8_rows_fits(a)) throw std::runtime_error("fp8 rows: shape");
  if (!a.a || !a.w || !a.c) throw std::runtime_error("fp8 gemm: null operand");
  if (fp8_rows_wide(a)) launch_fp8_rows_t<2>(a, st);
  else launch_fp8_rows_t<1>(a, st);
}

void launch_fp8_skinny(const Fp8GemmArgs& a0, hipStream_t st) {
  Fp8GemmArgs a = a0;
  if (a.M <= 0) return;
  if (a.K % 128 || a.K <= 0 || a.N <= 0) throw std::runtime_error("fp8 gemm: K % 128");
  if (!a.a || !a.w || !a.c) throw std::runtime_error("fp8 gemm: null operand");
  const bool f32s = a.sa32 != nullptr;
  if (f32s ? !a.sw32 : (!a.sa8 || !a.sw8)) throw std::runtime_error("fp8 gemm: scales");
  a.rows_cap = std::min(a.M, DN_MAXROWS);
  const size_t lds = size_t(a.rows_cap) * (a.K + DN_PAD) + size_t(a.rows_cap) * (a.K / 128) * (f32s ? 4 : 1);
  const dim3 grid(cdiv(cdiv(size_t(a.N), 16), DN_WAVES * DN_TN), cdiv(size_t(a.M), size_t(a.rows_cap)));
  if (f32s) {
    if (lds > 65536)
      UH_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(&fp8_skinny_kernel<true>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)));
    fp8_skinny_kernel<true><<<grid, DN_NT, lds, st>>>(a);
  } else {
    if (lds > 65536)
      UH_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(&fp8_skinny_kernel<false>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)));
    fp8_skinny_kernel<false><<<grid, DN_NT, lds, st>>>(a);
  }
  UH_CHECK_LAUNCH();
}

void launch_fp8_gemv(const Fp8GemmArgs& a, hipStream_t st, const Fp8Parts* parts) {
  if (a.M <= 0) return;
  if (a.M > 64) throw std::runtime_error("fp8 gemv: M > 64");
  Fp8Parts pp{};
  if (parts) {
    pp = *parts;
    if (pp.n < 1 || pp.n > 3 || a.sa32 || !a.sa8) throw std::runtime_error("fp8 gemv parts: 1..3 ranges, e8m0 scales");
    pp.t0[0] = 0;
    for (int i = 0; i < pp.n; ++i) {
      if (!pp.w[i] || !pp.sw[i] || !pp.c[i] || pp.N[i] <= 0) throw std::runtime_error("fp8 gemv parts: null part");
      pp.t0[i + 1] = pp.t0[i] + int(cdiv(size_t(pp.N[i]), 16));
    }
  } else if (a.N <= 0 || !a.w || !a.c) {
    throw std::runtime_error("fp8 gemm: null operand");
  }
  if (a.K % 128 || a.K <= 0) throw std::runtime_error("fp8 gemm: K % 128");
  if (!a.a) throw std::runtime_error("fp8 gemm: null operand");
  const bool f32s = a.sa32 != nullptr;
  if (!parts && (f32s ? !a.sw32 : (!a.sa8 || !a.sw8))) throw std::runtime_error("fp8 gemm: scales");
  if (f32s) launch_fp8_gemv_t<true>(a, st, pp);
  else launch_fp8_gemv_t<false>(a, st, pp);
}

// e2m1 fake quantization in place (the reference's ref_elem.hip:43-59): per block of `block` values, amax floored at
// 6 * 2^-126, sc = 2^ceil(log2(amax / 6)), x = bf16(e2m1(clamp(x / sc, +-6)) * sc) with the e2m1 rounding to nearest,
// ties to the even code. A thread per block, 8 values per 16-byte access (ldx % 8 == 0 on the host; other strides use
// 2-byte accesses); not a hot path (the attention indexer's operand).
__device__ __forceinline__ float round_e2m1_dev(float x) {
  const float a = fabsf(x);
  float r;
  if (a <= 0.25f) r = 0.0f;
  else if (a < 0.75f) r = 0.5f;
  else if (a <= 1.25f) r = 1.0f;
  else if (a < 1.75f) r = 1.5f;
  else if (a <= 2.5f) r = 2.0f;
  else if (a < 3.5f) r = 3.0f;
  else if (a <= 5.0f) r = 4.0f;
  else r = 6.0f;
  return x < 0.0f ? -r : r;
}
template <bool VEC>
__global__ __launch_bounds__(256) void fake_quant_fp4_kernel(bf16* x, int ldx, int rows, int cols, int block) {
  const int nb = cols / block;
  const size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x;
  if (i >= size_t(rows) * nb) return;
  bf16* xr = x + (i / nb) * size_t(ldx) + (i % nb) * size_t(block);
  float amax = 0.0f;
  if constexpr (VEC) {
    for (int c = 0; c < block; c += 8) {
      const uint4 v = *reinterpret_cast<const uint4*>(xr + c);
      const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int t = 0; t < 8; ++t) amax = fmaxf(amax, fabsf(bf16_to_f32(uint16_t(w4[t / 2] >> (16 * (t % 2))))));
    }
  } else {
    for (int c = 0; c < block; ++c) amax = fmaxf(amax, fabsf(bf16_to_f32(xr[c])));
  }
  amax = fmaxf(amax, 6.0f * 1.1754943508222875e-38f);  // 6 * 2^-126
  const float sc = e8m0_to_f32(pow2_ceil_e8m0(amax * (1.0f / 6.0f)));
  const auto q = [&](uint16_t v) {
    return f32_to_bf16(round_e2m1_dev(fminf(fmaxf(bf16_to_f32(v) / sc, -6.0f), 6.0f)) * sc);
  };
  if constexpr (VEC) {
    for (int c = 0; c < block; c += 8) {
      const uint4 v = *reinterpret_cast<const uint4*>(xr + c);
      const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
      uint32_t o[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) o[t] = uint32_t(q(uint16_t(w4[t]))) | (uint32_t(q(uint16_t(w4[t] >> 16))) << 16);
      *reinterpret_cast<uint4*>(xr + c) = uint4{o[0], o[1], o[2], o[3]};
    }
  } else {
    for (int c = 0; c < block; ++c) xr[c] = q(xr[c]);
  }
}

// ---- entry points ---------------------------------------------------------------------------------------------------
void fake_quant_fp4(bf16* x, int ldx, int rows, int cols, int block, hipStream_t st) {
  if (rows <= 0 || cols <= 0) return;
  if (block <= 0 || block % 8 || cols % block || ldx < cols || !x)
    throw std::runtime_error("fake_quant_fp4: block % 8, cols % block, ldx >= cols");
  const size_t n = size_t(rows) * (cols / block);
  const bool vec = ldx % 8 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
  if (vec) fake_quant_fp4_kernel<true><<<cdiv(n, 256), 256, 0, st>>>(x, ldx, rows, cols, block);
  else fake_quant_fp4_kernel<false><<<cdiv(n, 256), 256, 0, st>>>(x, ldx, rows, cols, block);
  UH_CHECK_LAUNCH();
}
void act_quant_fp8(const bf16* x, int ldx, uint8_t* q, uint8_t* s, int rows, int cols, int block, hipStream_t st) {
  launch_act_quant<0>(x, ldx, q, s, rows, cols, block, st);
}
void fake_quant_fp8(bf16* x, int ldx, int rows, int cols, int block, hipStream_t st) {
  launch_act_quant<1>(x, ldx, nullptr, nullptr, rows, cols, block, st);
}
void act_quant_fp8_f32s(const bf16* x, int ldx, uint8_t* q, float* s, int rows, int cols, int block, hipStream_t st) {
  launch_act_quant<2>(x, ldx, q, s, rows, cols, block, st);
}

void gemm_a8w4(const uint8_t* a, const uint8_t* sa, const uint8_t* w, const uint8_t* sw, bf16* c, int ldc, int M,
               int N, int K, hipStream_t st) {
  if (M <= 0) return;
  if (K % 128) throw std::runtime_error("gemm_a8w4: K % 128");
  gemm_a8w4_ref_kernel<false><<<dim3(cdiv(size_t(N), 256), unsigned(M)), 256, 0, st>>>(a, sa, w, sw, c, ldc, M, N, K);
  UH_CHECK_LAUNCH();
}
void gemm_a8w4_tiled(const uint8_t* a, const uint8_t* sa, const uint8_t* w, const uint8_t* sw, bf16* c, int ldc,
                     int M, int N, int K, hipStream_t st) {
  if (M <= 0) return;
  if (K % 128 || N % 16) throw std::runtime_error("gemm_a8w4_tiled: K % 128, N % 16");
  gemm_a8w4_ref_kernel<true><<<dim3(cdiv(size_t(N), 256), unsigned(M)), 256, 0, st>>>(a, sa, w, sw, c, ldc, M, N, K);
  UH_CHECK_LAUNCH();
}

void gemm_w8a8(const uint8_t* a, const uint8_t* sa, const uint8_t* w, const uint8_t* sw, bf16* c, int ldc, int M,
               int N, int K, hipStream_t st) {
  Fp8GemmArgs g{};
  g.a = a;
  g.sa8 = sa;
  g.w = w;
  g.sw8 = sw;
  g.c = c;
  g.ldc = ldc;
  g.M = M;
  g.N = N;
  g.K = K;
  launch_fp8_gemm(g, st);
}
void gemm_w8a8_wmma(const uint8_t* a, const uint8_t* sa, const uint8_t* w, const uint8_t* sw, bf16* c, int ldc,
                    int M, int N, int K, hipStream_t st) {
  gemm_w8a8(a, sa, w, sw, c, ldc, M, N, K, st);
}
void gemv_w8a8(const uint8_t* a, const uint8_t* sa, const uint8_t* w, const uint8_t* sw, bf16* c, int ldc, int M,
               int N, int K, hipStream_t st) {
  if (M > kGemvRowsCap) throw std::runtime_error("gemv_w8a8: M > 32");
  Fp8GemmArgs g{};
  g.a = a;
  g.sa8 = sa;
  g.w = w;
  g.sw8 = sw;
  g.c = c;
  g.ldc = ldc;
  g.M = M;
  g.N = N;
  g.K = K;
  launch_fp8_gemm(g, st);
}
void gemm_fp8_f32s_x(const bf16* x, int ldx, const uint8_t* w, const float* sw, bf16* c, int ldc, int M, int N,
                     int K, hipStream_t st) {
  if (M <= 0) return;
  if (M > 16) throw std::runtime_error("gemm_fp8_f32s_x: M <= 16");
  if (K % 128 || K <= 0 || N <= 0) throw std::runtime_error("gemm_fp8_f32s_x: K % 128");
  if (!x || !w || !sw || !c) throw std::runtime_error("gemm_fp8_f32s_x: null operand");
  if (ldx < K || ldx % 8 || reinterpret_cast<uintptr_t>(x) % 16) throw std::runtime_error("gemm_fp8_f32s_x: x rows");
  if (ldc < N) throw std::runtime_error("gemm_fp8_f32s_x: ldc < N");
  if (size_t(M) * K * (1 + 4.0 / 128) > 128 * 1024) throw std::runtime_error("gemm_fp8_f32s_x: M * K > 126 KiB");
  Fp8GemmArgs g{};
  g.xa = x;
  g.ldx = ldx;
  g.w = w;
  g.sw32 = sw;
  g.c = c;
  g.ldc = ldc;
  g.M = M;
  g.N = N;
  g.K = K;
  launch_fp8_gemv_xq(g, st);
}
void gemm_fp8_f32s(const uint8_t* a, const float* sa, const uint8_t* w, const float* sw, bf16* c, int ldc, int M,
                   int N, int K, hipStream_t st) {
  Fp8GemmArgs g{};
  g.a = a;
  g.sa32 = sa;
  g.w = w;
  g.sw32 = sw;
  g.c = c;
  g.ldc = ldc;
  g.M = M;
  g.N = N;
  g.K = K;
  launch_fp8_gemm(g, st);
}


namespace {
Fp8Parts to_parts(const GemvPart* parts, int nparts) {
  if (!parts || nparts < 1 || nparts > GemvParts::kMax) throw std::runtime_error("gemv_w8a8_parts: 1..3 parts");
  Fp8Parts pp{};
  pp.n = nparts;
  for (int i = 0; i < nparts; ++i) {
    pp.w[i] = static_cast<const uint8_t*>(parts[i].w);
    pp.sw[i] = parts[i].sw;
    pp.c[i] = static_cast<uint16_t*>(parts[i].c);
    pp.ldc[i] = parts[i].ldc;
    pp.N[i] = parts[i].N;
  }
  return pp;
}
}  // namespace

void gemv_w8a8_parts(const uint8_t* a, const uint8_t* sa, const GemvPart* parts, int nparts, int M, int K,
                     hipStream_t st) {
  if (M > kGemvRowsCap) throw std::runtime_error("gemv_w8a8_parts: M > 32");
  const Fp8Parts pp = to_parts(parts, nparts);
  Fp8GemmArgs g{};
  g.a = a;
  g.sa8 = sa;
  g.M = M;
  g.K = K;
  launch_fp8_gemv(g, st, &pp);
}

void gemv_w8a8_glu(const uint8_t* a, const uint8_t* sa, const GemvPart* parts, int M, int K, float limit,
                   const GemvQuant& gq, hipStream_t st) {
  if (!parts || parts[0].N != parts[1].N || parts[0].N % 128)
    throw std::runtime_error("gemv_w8a8_glu: two parts of one width (% 128)");
  if (!gq.q || !gq.qs) throw std::runtime_error("gemv_w8a8_glu: null q / qs");
  gemv_w8a8_parts(a, sa, parts, 2, M, K, st);
  launch_swiglu_quant(static_cast<const uint16_t*>(parts[0].c), parts[0].ldc, static_cast<const uint16_t*>(parts[1].c),
                      parts[1].ldc, M, parts[0].N, limit, nullptr, gq.q, gq.qs, st);
}

int gemv_max_rows() { return 8; }
void gemm_force_skinny(int) {}

}  // namespace unholy::kernels
