// Grouped GEMM with fp8 weights, "mgk,grk->mgr": c[m][g][r] = bf16(sum_k a[m][g][k] * (e4m3 w[g R + r][k] *
// e8m0 sw[(g R + r) / 128][k / 128])). a bf16 [M, G, K], w e4m3 [G R, K], sw [ceil(G R / 128), K / 128],
// c bf16 [M, G, R]. The reference's wo_a projection (src/model/forward_ref.hip:1012-1022, dense_grouped_fp8w
// :577-582): the weights dequantize exactly to bf16 (an e4m3 value times a power of two), so every product is exact
// and only the fp32 summation order separates the kernels.
//
// Three entry points, as the reference has them:
//   gemm_grouped_fp8w       the reference order (ref_gemm.hip:116-125, :198-202 at G = K: one fp32 fmaf chain over k
//                           in order), a thread per output: bit-exact against the CPU oracle, not a fast path;
//   gemm_grouped_fp8w_wmma  the fast path: the row-tile kernel for M <= 384 (M <= 16: R % 32 == 0, K <= 8192;
//                           else R % 64 == 0, K <= 4096), the GEMV for other shapes up to M = 160, else the tiled
//                           MFMA GEMM;
//   gemv_grouped_fp8w       M <= 32 as the fast path, optionally followed by act_quant_fp8 of its outputs (GemvQuant).
//
// GEMV (bound: HBM, 32 MB of weights at the DSV4 shape G = 8, R = 1024, K = 4096): a workgroup per 16-column tile,
// its 8 waves splitting K in 128-input blocks, every load of a chunk issued before its first use; bf16 MFMA
// 16x16x32 on the activations as they are and the weights dequantized with the block scale folded in; the 8
// partial tiles added in LDS in wave order.
// Row tiles (M <= 384): a workgroup per 64 columns x 32 rows (M <= 16: 32 columns x 16 rows) over the whole of K, the
// activation rows staged once per workgroup in LDS (the GEMV reads them once per 16 columns), the weights held in
// registers up to four chunks ahead.
// GEMM (bound: MFMA at M = 4096): 128-row tiles of one group, 4 waves, 64-input stages in an LDS ring filled by direct
// global -> LDS loads (two workgroups per CU); bf16 MFMA 32x32x16. A wave's columns lie in one 128-row weight block
// and a stage in one 128-input block, so the weight scale is one value per stage, folded into the dequantization.
#include <stdexcept>
#include <type_traits>
#include <string>

#include "common.hpp"
#include "numerics.hpp"
#include "pipe.hpp"
#include "unholy/kernels/gemm_wmma.hpp"
#include "unholy/kernels/gemv.hpp"
#include "unholy/kernels/ref.hpp"

namespace unholy::kernels {

using namespace uh;
using namespace pipe;

namespace {

// ---- reference order ------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void grouped_fp8w_ref_kernel(const bf16* a, const uint8_t* w, const uint8_t* sw,
                                                               bf16* c, int M, int G, int R, int K) {
  const int n = blockIdx.x * 256 + threadIdx.x, m = blockIdx.y;
  if (n >= G * R) return;
  const int g = n / R, kbs = K / 128;
  const bf16* am = a + (size_t(m) * G + g) * K;
  const uint8_t* wn = w + size_t(n) * K;
  float acc = 0.0f;
  for (int k = 0; k < K; ++k)
    acc = fmaf(bf16_to_f32(am[k]), e4m3_to_f32(wn[k]) * e8m0_to_f32(sw[size_t(n / 128) * kbs + k / 128]), acc);
  c[size_t(m) * G * R + n] = f32_to_bf16(acc);
}

// ---- GEMV ------------------------------------------------------------------------------------------------------------
constexpr int GV_W = 8, GV_CHUNK = 4;

// Workgroup (blockIdx.x, blockIdx.y) = 16 columns x row chunk blockIdx.y of 16 MT rows: several chunks when M is
// above 16 MT (each chunk re-reads the tile's weights, from the Infinity Cache when the chunks run close together).
template <int MT>
__global__ __launch_bounds__(64 * GV_W) void grouped_fp8w_gemv_kernel(const bf16* a, const uint8_t* w,
                                                                      const uint8_t* sw, bf16* c, int M, int G, int R,
                                                                      int K) {
  __shared__ v4f red[GV_W][MT][64];
  const int KS = K / 128, N = G * R;
  a += size_t(blockIdx.y) * 16 * MT * G * K;
  c += size_t(blockIdx.y) * 16 * MT * N;
  M = min(16 * MT, M - int(blockIdx.y) * 16 * MT);
  const int tid = threadIdx.x, lane = tid & 63, nl = lane & 15, q4 = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n0 = blockIdx.x * 16, n = n0 + nl, grp = n0 / R;  // R % 16 == 0: the tile lies in one group
  const int per = (KS + GV_W - 1) / GV_W, b0 = min(KS, wave * per), b1 = min(KS, b0 + per);
  const uint8_t* wrow = w + size_t(n) * K + q4 * 32;
  const uint8_t* swrow = sw + size_t(n0 / 128) * KS;  // a 16-column tile lies in one 128-row block
  v4f acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  for (int kc = b0; kc < b1; kc += GV_CHUNK) {
    // Lane (nl, q4) holds inputs 32 q4 .. 32 q4 + 31 of each 128-input block: 32 codes of column n and 32 bf16 of
    // row nl (rows past M clamped, their products discarded).
    v4i b[GV_CHUNK][2], x[GV_CHUNK][MT][4];
    float swv[GV_CHUNK];
#pragma unroll
    for (int u = 0; u < GV_CHUNK; ++u) {
      const int kb = min(kc + u, b1 - 1);
      b[u][0] = *reinterpret_cast<gptr<v4i>>(as_global(wrow + kb * 128));
      b[u][1] = *reinterpret_cast<gptr<v4i>>(as_global(wrow + kb * 128 + 16));
      swv[u] = e8m0_to_f32(swrow[kb]);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const bf16* ap = a + (size_t(min(mt * 16 + nl, M - 1)) * G + grp) * K + kb * 128 + q4 * 32;
#pragma unroll
        for (int i = 0; i < 4; ++i) x[u][mt][i] = *reinterpret_cast<gptr<v4i>>(as_global(ap + 8 * i));
      }
    }
#pragma unroll
    for (int u = 0; u < GV_CHUNK; ++u) {
      if (kc + u >= b1) break;
      bf16x8 bf[4];
#pragma unroll
      for (int t = 0; t < 4; ++t)
        bf[t] = fp8x8_to_bf16(uint32_t(b[u][t / 2][2 * (t % 2)]), uint32_t(b[u][t / 2][2 * (t % 2) + 1]), swv[u]);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if (mt * 16 >= M) break;
        const bool live = mt * 16 + nl < M;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const bf16x8 af = live ? __builtin_bit_cast(bf16x8, x[u][mt][t]) : bf16x8{};
          acc[mt] = mfma_bf16(af, bf[t], acc[mt]);
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
    for (int v = 1; v < GV_W; ++v) s += red[v][wave][lane];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = wave * 16 + 4 * q4 + i;
      if (r < M) c[size_t(r) * N + n] = f32_to_bf16(s[i]);
    }
  }
}

// ---- row tiles, M <= 384 -----------------------------------------------------------------------------------------
// A workgroup per 64 columns (one group: R % 64 == 0) x 32 rows, the whole of K (<= 4,096), bf16 C written directly
// (M <= 16: 32 columns x 16 rows, K <= 8,192, 16 K parts of 2,048-input chunks; the parameters below):
// - 16 waves = 2 column halves x 8 K parts, 32 x 32 output tiles (bf16 MFMA 32x32x16); part p takes block p of every
//   1,024-input chunk;
// - a wave's weights for all (<= 4) chunks are loaded into registers up front, interleaved with the first two
//   activation chunks (issue order: scales, W0 A0 W1 A1 W2 W3, then A(c + 2) once chunk c is done), so chunk c starts
//   while the later weights stream; loads retire in order and each chunk waits for exactly the loads before its own;
// - the tile's activation rows go through a 2-slot LDS ring of chunks (32 rows x 1,024 bf16, 64 KB) by direct
//   global -> LDS loads; piece p (16 bytes) of row r sits at p ^ (r & 15), so the 16 rows of an MFMA operand pass
//   cover the 64 banks once (the 32-column form: each wave stages its own K part's 16 rows in its own ring and waits
//   for no other wave until the reduction);
// - the weights dequantize with the block scale folded in (exact); the 8 parts (16 in the 32-column form) are added
//   in LDS in part order by all 16 waves;
// - work item wi = column block x row tiles + row tile; XCD x takes the x-th eighth of the items, so the row tiles of
//   a column block share one L2 (the second reads the weights from it) and a group's activation rows sit in one L2.
// Against the GEMV (one 16-column tile per workgroup, every workgroup reading its rows from L2): the activation rows
// leave L2 once per 64 columns. DSV4 shape: 17.6 us against 45 us at M = 64; at M = 1 8.9 us against 10.8 us (the
// 32-column form: 256 workgroups, each wave's weights in flight at once).
constexpr int GR_SLOT = 64 * 1024, GR_MAXCH = 4;

// CH column halves of 32 (workgroup width 32 CH), TR staged rows (32, or 16 for M <= 16: the MFMA's rows 16-31 then
// read rows 0-15 again and are not stored); KP = 16 / CH K parts, chunks of KR = 128 KP inputs, a 64 KB slot either way.
template <int CH, int TR>
struct GroupedRows {
  static constexpr int KP = 16 / CH, KR = 128 * KP, PPR = KR / 8, W = 32 * CH;
  static_assert(TR * KR * 2 == GR_SLOT, "one chunk fills a slot");
};

// NCH = the chunk count, ceil((K / 128) / KP) (1..GR_MAXCH): a template parameter, so that the issue order and every
// counted wait are fixed at compile time and no branch depends on how many loads are outstanding.
template <int CH, int TR, int NCH>
__global__ __launch_bounds__(1024) void grouped_fp8w_rows_kernel(const bf16* a, const uint8_t* w, const uint8_t* sw,
                                                                 bf16* c, int M, int G, int R, int K) {
  using T = GroupedRows<CH, TR>;
  constexpr int KP = T::KP, KR = T::KR, PPR = T::PPR;
  extern __shared__ __align__(16) uint8_t smem[];
  static_assert(NCH >= 1 && NCH <= GR_MAXCH);
  static_assert(CH == 2 || TR == 16, "the per-wave activation loads cover 16 rows");
  const int N = G * R, KS = K / 128;  // the host launches NCH = ceil(KS / KP)
  const int nw = gridDim.x, lin = blockIdx.x;
  const int wi = nw % 8 ? lin : (lin & 7) * (nw >> 3) + (lin >> 3);
  const int RT = (M + TR - 1) / TR, rt = wi % RT, bx = wi / RT, row0 = rt * TR;
  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), chh = wave % CH, kh = wave / CH;
  const int col0 = bx * T::W, grp = col0 / R, n = col0 + chh * 32 + l32;
  // Weight load x (0..3) of a block: lane l reads 16 bytes of column row 16 (x >> 1) + l % 16 at byte 64 (x & 1) +
  // 16 (l >> 4), so a load covers 64 contiguous bytes of each of 16 rows (32 bytes of 32 rows in the MFMA's own
  // layout measured 2.6 us slower at the DSV4 shape). One lane-row swap per dword pair (loads 0 <-> 2, 1 <-> 3) then
  // leaves lane l with column l % 32: load x holds piece (16 bytes) 2 h + (x >> 1) + 4 (x & 1) of the block.
  const uint8_t* wld = w + size_t(col0 + chh * 32 + (lane & 15)) * K + (lane >> 4) * 16;
  const uint8_t* swrow = sw + size_t((col0 + chh * 32) / 128) * KS;  // 32 columns lie in one 128-row block
  const uint32_t lds0 = lds_addr(smem);
  // This wave's 4 direct loads of a chunk (rows past M repeat row M - 1; neither they nor the clamped inputs are
  // used).
  // - CH = 1 (16 rows): the wave's own K part, 16 rows x 128 inputs (4 KB), into its own 2-slot ring: load i covers
  //   rows 4i .. 4i + 3, lane j row 4i + j / 16 at piece (j % 16) ^ row, so a 16-lane pass of the MFMA's 16-byte
  //   reads (16 rows, one piece) covers the 64 banks once. No wave waits for another before the reduction: a wave
  //   computes its chunks as soon as its own loads land while the others still stream.
  // - CH = 2 (32 rows, the two column halves of a K part read the same activations): 1 KB pieces q = 4 wave + i of
  //   the shared 64 KB chunk slot, read after a barrier.
  uint32_t rowoff[4];
  int pin[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (CH == 1) {
      const int r = 4 * i + (lane >> 4);
      rowoff[i] = uint32_t(min(row0 + r, M - 1) * G + grp) * uint32_t(K) * 2u;
      pin[i] = ((lane & 15) ^ r) * 8;
    } else {
      const int slot = (wave * 4 + i) * 64 + lane, r = slot / PPR;
      rowoff[i] = uint32_t(min(row0 + r, M - 1) * G + grp) * uint32_t(K) * 2u;
      pin[i] = ((slot % PPR) ^ (r & 15)) * 8;
    }
  }
  const auto issue_a = [&](int ch) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (CH == 1)
        dma16(a, rowoff[i] + uint32_t(min(ch * KP + kh, KS - 1) * 128 + pin[i]) * 2u,
              lds0 + uint32_t((wave * 2 + (ch & 1)) * 4096 + i * 1024));
      else
        dma16(a, rowoff[i] + uint32_t(min(ch * KR + pin[i], K - 8)) * 2u,
              lds0 + uint32_t((ch & 1) * GR_SLOT + (wave * 4 + i) * 1024));
    }
  };
  v4i b[NCH][4];
  const auto load_w = [&](int u) {
    const uint8_t* p = wld + min(u * KP + kh, KS - 1) * 128;
#pragma unroll
    for (int x = 0; x < 4; ++x) b[u][x] = vload16(p + (x >> 1) * 16 * K + (x & 1) * 64);
  };
  // Issue order: the wave's block scales (lane u: chunk u), W0 A0 W1 A1 W2 W3, then A(c + 2) once chunk c is done.
  // Loads retire in order, so chunk c starts while the later chunks stream.
  uint32_t sv = vload_u8(swrow + min(min(lane, GR_MAXCH - 1) * KP + kh, KS - 1));
  load_w(0);
  issue_a(0);
  if constexpr (NCH > 1) {
    load_w(1);
    issue_a(1);
  }
  if constexpr (NCH > 2) load_w(2);
  if constexpr (NCH > 3) load_w(3);
  const int r = l32 & (TR - 1);
  v16f_t acc = v16f_t{};
  const auto chunk = [&](auto ich) {
    constexpr int ch = decltype(ich)::value;
    // Chunk ch, its weights and the scales have landed when only the loads issued after A(ch) are pending (4 per
    // group): ch = 0: W1 A1 W2 W3; ch = 1: W2 W3 A2; ch = 2: A3; each where it exists.
    constexpr int later = 4 * (ch == 0   ? (1 < NCH) * 2 + (2 < NCH) + (3 < NCH)
                               : ch == 1 ? (2 < NCH) * 2 + (3 < NCH)
                               : ch == 2 ? (3 < NCH)
                                         : 0);
    wait_vm<later>();
    vlanded(b[ch]);
    vlanded(sv);
    if constexpr (CH == 1) asm volatile("" ::: "memory");  // the wave's own activation pieces have landed in LDS
    else __syncthreads();                                    // every wave's part of chunk ch has landed
    if (ch * KP + kh < KS) {
      const uint8_t* sl = CH == 1 ? smem + (wave * 2 + (ch & 1)) * 4096 : smem + (ch & 1) * GR_SLOT;
      const float swc = __uint_as_float(uint32_t(__builtin_amdgcn_readlane(int(sv), ch)) << 23);
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
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int x = j >> 1;
        const bf16x8 bf = fp8x8_to_bf16(uint32_t(b[ch][x][2 * (j & 1)]), uint32_t(b[ch][x][2 * (j & 1) + 1]), swc);
        const int q = 2 * (2 * h + (x >> 1) + 4 * (x & 1)) + (j & 1);  // the block's piece of this MFMA
        const bf16x8 af = CH == 1
            ? __builtin_bit_cast(bf16x8, *reinterpret_cast<const v4i*>(sl + (r * 16 + (q ^ r)) * 16))
            : __builtin_bit_cast(bf16x8, *reinterpret_cast<const v4i*>(sl + (r * PPR + ((kh * 16 + q) ^ (r & 15))) * 16));
        acc = mfma32_bf16(af, bf, acc);
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
  // The KP parts added in part order through LDS, shared by all waves: wave (chh, kh) adds elements CH kh ..
  // CH kh + CH - 1 of its column half's lanes. Lane stride 18 floats for 8-byte reads (CH 2), 17 for 4-byte ones
  // (CH 1): a half-wave's reads cover the 64 banks once.
  __syncthreads();
  float* red = reinterpret_cast<float*>(smem);
  constexpr int LS = CH == 2 ? 18 : 17;
  float* mine = red + ((kh * CH + chh) * 64 + lane) * LS;
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
  for (int e = 0; e < CH; ++e) sum[e] = red[(chh * 64 + lane) * LS + CH * kh + e];
#pragma unroll
  for (int q = 1; q < KP; ++q)
#pragma unroll
    for (int e = 0; e < CH; ++e) sum[e] += red[((q * CH + chh) * 64 + lane) * LS + CH * kh + e];
  // Element i of lane (l32, h) is row 8 (i / 4) + 4 h + i % 4 of the tile, column l32 of the half.
#pragma unroll
  for (int e = 0; e < CH; ++e) {
    const int i = CH * kh + e, rr = 8 * (i / 4) + 4 * h + (i % 4);
    if (rr < TR && row0 + rr < M) c[size_t(row0 + rr) * N + n] = f32_to_bf16(sum[e]);
  }
}

// M <= 16: 32-column workgroups of 16 staged rows (256 workgroups at the DSV4 shape, every wave's weights in flight at
// once); 16 < M <= GR_MAXM: 64-column workgroups of 32-row tiles. At the DSV4 shape the row tiles ran 44 / 58 / 86 us
// at M = 192 / 256 / 384 against 100-106 us for the tiled GEMM (128 workgroups or fewer there), which wins from
// M = 512 on (107 against 116 us).
constexpr int GR_MAXM = 384;
bool rows_fits(int M, int G, int R, int K) {
  if (M < 1 || M > GR_MAXM || size_t(M) * G * K * 2 >= (size_t(1) << 32)) return false;
  return M <= 16 ? R % 32 == 0 && K <= GR_MAXCH * GroupedRows<1, 16>::KR
                 : R % 64 == 0 && K <= GR_MAXCH * GroupedRows<2, 32>::KR;
}
template <int CH, int TR>
void launch_rows_t(const bf16* a, const uint8_t* w, const uint8_t* sw, bf16* c, int M, int G, int R, int K,
                   hipStream_t st) {
  const size_t lds = 2 * size_t(GR_SLOT);
  const int nch = (K / 128 + GroupedRows<CH, TR>::KP - 1) / GroupedRows<CH, TR>::KP;  // 1..GR_MAXCH (rows_fits)
  auto* kern = nch == 1   ? &grouped_fp8w_rows_kernel<CH, TR, 1>
               : nch == 2 ? &grouped_fp8w_rows_kernel<CH, TR, 2>
               : nch == 3 ? &grouped_fp8w_rows_kernel<CH, TR, 3>
                          : &grouped_fp8w_rows_kernel<CH, TR, 4>;
  UH_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                               int(lds)));
  kern<<<dim3(unsigned(G * R / GroupedRows<CH, TR>::W * ((M + TR - 1) / TR))), 1024, lds, st>>>(a, w, sw, c, M, G, R,
                                                                                                 K);
  UH_CHECK_LAUNCH();
}
void launch_rows(const bf16* a, const uint8_t* w, const uint8_t* sw, bf16* c, int M, int G, int R, int K,
                 hipStream_t st) {
  if (M <= 16) launch_rows_t<1, 16>(a, w, sw, c, M, G, R, K, st);
  else launch_rows_t<2, 32>(a, w, sw, c, M, G, R, K, st);
}

// ---- tiled GEMM ------------------------------------------------------------------------------------------------------
// Tile 128 rows x TN columns of one group, 4 waves of 64 rows x TN / 2 columns (TN / 64 MFMA blocks of 32 x 32 across
// each wave's columns), 64-input stages. TN 256 (R % 256 == 0): 2 slots of 32 KB, 32 MFMAs per wave per stage; TN 128:
// 3 slots of 24 KB, 16 MFMAs per stage. Either way under 80 KB of LDS, two workgroups per CU.
template <int TN>
struct GroupedTile {
  static constexpr int A = 128 * 128, B = TN * 64, STAGE = A + B, S = TN == 256 ? 2 : 3, RING = S * STAGE;
  static constexpr int CB = TN / 64, OPS = 4 + TN / 64;  // MFMA column blocks per wave; direct loads per wave per stage
  static constexpr int LDC = TN + 8;
  static constexpr size_t lds() { return RING > 128 * LDC * 2 ? size_t(RING) : size_t(128) * LDC * 2; }
};

// XOR swizzle of a 64-byte row (4 pieces of 16 bytes): an operand read's pass covers 16 consecutive rows starting at
// a multiple of 16 at one piece, and (n % 4) * 4 + (p ^ ((n >> 2) & 3)) modulo 16 differs across them, so the pass
// touches each of the 64 banks once.
__device__ __forceinline__ int swz64(int n) { return (n >> 2) & 3; }

template <int TN>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void grouped_fp8w_tiled_kernel(
    const bf16* a, const uint8_t* w, const uint8_t* sw, bf16* c, int M, int G, int R, int K) {
  using T = GroupedTile<TN>;
  extern __shared__ __align__(16) uint8_t smem[];
  int bx, by;
  tile_block(gridDim.x, bx, by);
  const int row0 = by * 128;
  if (row0 >= M) return;  // padding of the grid's row-tile count
  const int KS = K / 64, N = G * R, Mt = min(128, M - row0), col0 = bx * TN, grp = col0 / R;
  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rh = wave & 1, ch = wave >> 1;
  const uint32_t lds0 = lds_addr(smem);
  // Per-lane load offsets (bytes; constant over the stages). A: 128-byte row pieces (64 bf16 of a stage) of row r
  // of the group, rows past the tile repeating its last; B: 64-byte row pieces of weight row col0 + n.
  uint32_t aoff[4], boff[T::CB];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int slot = (wave * 4 + i) * 64 + lane, r = slot >> 3, p = (slot & 7) ^ lds_swz(r);
    aoff[i] = uint32_t(min(r, Mt - 1) * G + grp) * uint32_t(2 * K) + uint32_t(p * 16);
  }
#pragma unroll
  for (int i = 0; i < T::CB; ++i) {
    const int slot = (wave * T::CB + i) * 64 + lane, n = slot >> 2, p = (slot & 3) ^ swz64(n);
    boff[i] = uint32_t(n) * uint32_t(K) + uint32_t(p * 16);
  }
  const uint8_t* abase = reinterpret_cast<const uint8_t*>(a + size_t(row0) * G * K);
  const uint8_t* wbase = w + size_t(col0) * K;
  // The wave's TN / 2 columns lie in one 128-row weight block: one scale per stage.
  const uint8_t* swrow = sw + size_t((col0 + ch * (TN / 2)) / 128) * (K / 128);
  const auto issue = [&](int s) {
    const uint32_t st = lds0 + uint32_t((s % T::S) * T::STAGE);
#pragma unroll
    for (int i = 0; i < 4; ++i) dma16(abase + s * 128, aoff[i], st + uint32_t(wave * 4 + i) * 1024);
#pragma unroll
    for (int i = 0; i < T::CB; ++i) dma16(wbase + s * 64, boff[i], st + uint32_t(T::A + (wave * T::CB + i) * 1024));
  };
  for (int j = 0; j < T::S - 1 && j < KS; ++j) issue(j);

  const int rb_live = __builtin_amdgcn_readfirstlane(min(2, max(0, (Mt - rh * 64 + 31) / 32)));
  v16f_t acc[2][T::CB];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int cb = 0; cb < T::CB; ++cb) acc[rb][cb] = v16f_t{};

  // The wave's live 32-row blocks as a compile-time count (2 but in a partial last row tile): no branch in the stage
  // loop.
  const auto stages = [&](auto rbl) {
    constexpr int RBL = decltype(rbl)::value;
    for (int s = 0; s < KS; ++s) {
      // This wave's part of stage s has landed when at most its loads of the later stages issued (S - 2 at most) are
      // pending.
      if (T::S == 3 && s + 1 < KS) wait_vm<T::OPS>();
      else wait_vm<0>();
      __syncthreads();  // every wave's part has landed; slot (s - 1) % S is free
      if (s + T::S - 1 < KS) issue(s + T::S - 1);
      const uint8_t* stb = smem + (s % T::S) * T::STAGE;
      const float swv = e8m0_to_f32(swrow[s >> 1]);
      // MFMA step t (16 inputs): lane half h supplies inputs 32 h + 8 t .. + 7 of the stage, on both sides.
      v4i bq[T::CB][2];
#pragma unroll
      for (int cb = 0; cb < T::CB; ++cb) {
        const int n = ch * (TN / 2) + cb * 32 + l32;
#pragma unroll
        for (int x = 0; x < 2; ++x)
          bq[cb][x] = *reinterpret_cast<const v4i*>(stb + T::A + (n * 4 + ((2 * h + x) ^ swz64(n))) * 16);
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        bf16x8 bf[T::CB];
#pragma unroll
        for (int cb = 0; cb < T::CB; ++cb)
          bf[cb] = fp8x8_to_bf16(uint32_t(bq[cb][t >> 1][(t & 1) * 2]), uint32_t(bq[cb][t >> 1][(t & 1) * 2 + 1]), swv);
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
          if (rb >= RBL) break;
          const int r = rh * 64 + rb * 32 + l32;
          const bf16x8 af =
              __builtin_bit_cast(bf16x8, *reinterpret_cast<const v4i*>(stb + (r * 8 + ((4 * h + t) ^ lds_swz(r))) * 16));
#pragma unroll
          for (int cb = 0; cb < T::CB; ++cb) acc[rb][cb] = mfma32_bf16(af, bf[cb], acc[rb][cb]);
        }
      }
    }
  };
  if (rb_live == 2) stages(std::integral_constant<int, 2>{});
  else if (rb_live == 1) stages(std::integral_constant<int, 1>{});
  else stages(std::integral_constant<int, 0>{});

  // ---- epilogue through LDS: 128 x TN bf16, then 16-byte row stores
  __syncthreads();
  uint16_t* sc = reinterpret_cast<uint16_t*>(smem);
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int cb = 0; cb < T::CB; ++cb)
#pragma unroll
      for (int i = 0; i < 16; ++i)
        sc[(rh * 64 + rb * 32 + 8 * (i / 4) + 4 * h + (i % 4)) * T::LDC + ch * (TN / 2) + cb * 32 + l32] =
            f32_to_bf16(acc[rb][cb][i]);
  __syncthreads();
  for (int e = tid; e < Mt * (TN / 8); e += 256) {
    const int r = e / (TN / 8), c8 = (e % (TN / 8)) * 8;
    *reinterpret_cast<uint4*>(c + size_t(row0 + r) * N + col0 + c8) = *reinterpret_cast<const uint4*>(sc + r * T::LDC + c8);
  }
}

void check_args(const char* name, const bf16* a, const uint8_t* w, const uint8_t* sw, const bf16* c, int M, int G,
                int R, int K) {
  if (M < 0 || G <= 0 || R <= 0 || K <= 0 || K % 128) throw std::runtime_error(std::string(name) + ": K % 128");
  if (!a || !w || !sw || !c) throw std::runtime_error(std::string(name) + ": null operand");
}

void launch_ref(const bf16* a, const uint8_t* w, const uint8_t* sw, bf16* c, int M, int G, int R, int K,
                hipStream_t st) {
  grouped_fp8w_ref_kernel<<<dim3(unsigned(cdiv(size_t(G) * R, 256)), unsigned(M)), 256, 0, st>>>(a, w, sw, c, M, G,
                                                                                                 R, K);
  UH_CHECK_LAUNCH();
}

// The GEMV for up to 160 rows (32-row chunks side by side) where the row-tile kernel does not take the shape, the tiled
// GEMM above: at the DSV4 shape M = 64 the GEMV ran 46 us as two chunks, the tiled kernel 69 us (64 workgroups).
constexpr int GV_MAX_ROWS = 160;
bool gemv_fits(int M, int R) { return M <= GV_MAX_ROWS && R % 16 == 0; }
void launch_gemv(const bf16* a, const uint8_t* w, const uint8_t* sw, bf16* c, int M, int G, int R, int K,
                 hipStream_t st) {
  const unsigned tiles = unsigned(size_t(G) * R / 16);
  if (M <= 16) grouped_fp8w_gemv_kernel<1><<<dim3(tiles), 64 * GV_W, 0, st>>>(a, w, sw, c, M, G, R, K);
  else grouped_fp8w_gemv_kernel<2><<<dim3(tiles, unsigned(cdiv(M, 32))), 64 * GV_W, 0, st>>>(a, w, sw, c, M, G, R, K);
  UH_CHECK_LAUNCH();
}

// 32-bit DMA offsets: a tile's rows span 128 G K bf16 from its base.
bool tiled_fits(int G, int R, int K) { return R % 128 == 0 && size_t(128) * G * K * 2 < (size_t(1) << 32); }
template <int TN>
void launch_tiled_t(const bf16* a, const uint8_t* w, const uint8_t* sw, bf16* c, int M, int G, int R, int K,
                    hipStream_t st) {
  const size_t lds = GroupedTile<TN>::lds();
  auto* kern = &grouped_fp8w_tiled_kernel<TN>;
  UH_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                               int(lds)));
  kern<<<tile_grid(G * R / TN, (M + 127) / 128), 256, lds, st>>>(a, w, sw, c, M, G, R, K);
  UH_CHECK_LAUNCH();
}
void launch_tiled(const bf16* a, const uint8_t* w, const uint8_t* sw, bf16* c, int M, int G, int R, int K,
                  hipStream_t st) {
  // 256-column tiles once they leave more than 256 workgroups; before that twice the workgroups of 128 columns win
  // (DSV4 shape: 88 / 91 / 101 us at M = 512 / 768 / 1024 against 105 / 108 / 114; 157 against 197 us at M = 2048).
  if (R % 256 == 0 && size_t((M + 127) / 128) * (size_t(G) * R / 256) > 256)
    launch_tiled_t<256>(a, w, sw, c, M, G, R, K, st);
  else
    launch_tiled_t<128>(a, w, sw, c, M, G, R, K, st);
}

}  // namespace

void gemm_grouped_fp8w(const bf16* a, const uint8_t* w, const uint8_t* sw, bf16* c, int M, int G, int R, int K,
                       hipStream_t st) {
  check_args("gemm_grouped_fp8w", a, w, sw, c, M, G, R, K);
  if (M == 0) return;
  launch_ref(a, w, sw, c, M, G, R, K, st);
}

void gemm_grouped_fp8w_wmma(const bf16* a, const uint8_t* w, const uint8_t* sw, bf16* c, int M, int G, int R, int K,
                            hipStream_t st) {
  check_args("gemm_grouped_fp8w_wmma", a, w, sw, c, M, G, R, K);
  if (M == 0) return;
  if (rows_fits(M, G, R, K)) launch_rows(a, w, sw, c, M, G, R, K, st);
  else if (gemv_fits(M, R)) launch_gemv(a, w, sw, c, M, G, R, K, st);
  else if (tiled_fits(G, R, K)) launch_tiled(a, w, sw, c, M, G, R, K, st);
  else launch_ref(a, w, sw, c, M, G, R, K, st);  // shapes the fast kernels do not tile (R % 128 != 0)
}

void gemv_grouped_fp8w(const bf16* a, const uint8_t* w, const uint8_t* sw, bf16* c, int M, int G, int R, int K,
                       hipStream_t st, const GemvQuant& gq) {
  check_args("gemv_grouped_fp8w", a, w, sw, c, M, G, R, K);
  if (M > 32) throw std::runtime_error("gemv_grouped_fp8w: M > 32");  // the reference's bound (gemv.hip:653)
  if (gq.q && (!gq.qs || (size_t(G) * R) % 128)) throw std::runtime_error("gemv_grouped_fp8w: quantization shape");
  if (M == 0) return;
  if (rows_fits(M, G, R, K)) launch_rows(a, w, sw, c, M, G, R, K, st);
  else if (gemv_fits(M, R)) launch_gemv(a, w, sw, c, M, G, R, K, st);
  else launch_ref(a, w, sw, c, M, G, R, K, st);
  // act_quant_fp8 (block 128) of the bf16 outputs, the values the reference's last blocks quantize (a second launch
  // here instead of its per-segment counters, which stay zero).
  if (gq.q) act_quant_fp8(c, G * R, gq.q, gq.qs, M, G * R, 128, st);
}

}  // namespace unholy::kernels
