// Dense fp8 GEMM for larger M: C[M, N] (bf16) = A[M, K] (e4m3) x W[N, K]^T (e4m3), per-128 scales (e8m0 for
// gemm_w8a8, the reference's ref_gemm.hip:130-137 / gemm_wmma.hip:51-183; fp32 for the 1x128 / 128x128 format of
// tools/ref/oracle/kernel.py:81-118).
//
// Workgroup = 256 threads, 128 rows x TN columns (TN = 128, or 64 while 128-column tiles would make fewer than 256
// workgroups); wave w owns rows 64 (w & 1) .. + 63 and columns TN / 2 (w >> 1) .. + TN / 2 - 1.
// Per 128-input stage a 2-slot LDS ring holds
//   A 16 KB: row r's 16-byte piece p at slot r * 8 + (p ^ lds_swz(r)),
//   B TN x 128 B: column n's 16-byte piece p at slot n * 8 + (p ^ lds_swz(n)) (W is row-major like A),
//   S 512 B: fp32 activation scales of the 128 rows (fp32 form only, one gathered dword per row),
// filled by direct global -> LDS loads: stage s + 1 is issued right after stage s's barrier. A workgroup stays under
// 80 KB of LDS, so two share a CU and one's barriers and operand waits overlap the other's MFMAs.
// Both operands are dequantized exactly to bf16 at the LDS read and multiplied on the 32x32x16 bf16 MFMA. e8m0
// scales are folded into the conversions (exact) and the MFMA accumulates across blocks; with fp32 scales each
// block's MFMA chain starts from zero and is folded as acc += raw * (sa * sw), the reference's order of scaling.
#include <type_traits>
#include <stdexcept>

#include "common.hpp"
#include "numerics.hpp"
#include "fp8_internal.hpp"
#include "pipe.hpp"

namespace unholy::kernels {

using namespace uh;
using namespace pipe;

namespace {

// TN output columns per workgroup: 128, or 64 where 128-column tiles would leave too few workgroups (each wave then
// owns 64 rows x 32 columns).
template <int TN>
struct FpTile {
  static constexpr int S = 2, A = 128 * 128, B = TN * 128, SA = 128 * 4, STAGE = A + B + SA, RING = S * STAGE;
  static constexpr int LDC = TN + 8, CB = TN / 64, BL = TN / 32;  // column blocks per wave, B loads per wave
  static_assert(128 * LDC * 2 <= RING, "the bf16 C tile reuses the ring");
  static size_t lds(int K, bool f32s) { return size_t(RING) + size_t(4 + (f32s ? 0 : 128)) * (K / 128); }
};

template <bool F32S, int TN>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void fp8_tiled_kernel(Fp8GemmArgs a) {
  using T = FpTile<TN>;
  constexpr int FT_S = T::S, FT_A = T::A, FT_B = T::B, FT_STAGE = T::STAGE, FT_RING = T::RING, FT_LDC = T::LDC;
  constexpr int CB = T::CB;
  extern __shared__ __align__(16) uint8_t smem[];
  int bx, by;
  tile_block(gridDim.x, bx, by);
  const int K = a.K, KS = K / 128, M = a.M;
  const int row0 = by * 128;
  if (row0 >= M) return;  // padding of the grid's row-tile count
  const int Mt = min(128, M - row0), col0 = bx * TN;
  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rh = wave & 1, ch = wave >> 1;
  const uint32_t lds0 = lds_addr(smem);
  // After the ring: the weight scales of the workgroup's 128-column block [KS] as fp32, then (e8m0 form) the
  // activation scales [KS][128]. Copied once, so the stage loop issues no global loads besides the ring's.
  float* const sw_lds = reinterpret_cast<float*>(smem + FT_RING);
  uint8_t* const sa_lds = smem + FT_RING + 4 * KS;

  // Per-lane load offsets (constant over the stages). Rows past the tile repeat its last row (never stored).
  uint32_t aoff[4], boff[T::BL];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int slot = (wave * 4 + i) * 64 + lane, r = slot >> 3, p = (slot & 7) ^ lds_swz(r);
    aoff[i] = uint32_t(min(r, Mt - 1)) * uint32_t(K) + uint32_t(p * 16);
  }
#pragma unroll
  for (int i = 0; i < T::BL; ++i) {  // columns: the same slot geometry
    const int slot = (wave * T::BL + i) * 64 + lane, r = slot >> 3, p = (slot & 7) ^ lds_swz(r);
    boff[i] = uint32_t(r) * uint32_t(K) + uint32_t(p * 16);
  }
  // fp32 scales: the fold's factor sa[row] * sw (the reference's order, raw * (sa * sw)) for each stage's 128 rows is
  // formed once, by waves 0 and 1 (rows 64 w + lane) one stage ahead: the next stage's sa is loaded into a register
  // and, at the end of the current stage, multiplied and written into that stage's slot; the fold of every wave then
  // reads the products instead of forming 32 of them per lane.
  const float* sarow = F32S ? a.sa32 + size_t(row0 + min((wave & 1) * 64 + lane, Mt - 1)) * KS : nullptr;
  const float* swcol = F32S ? a.sw32 + size_t(col0 / 128) * KS : nullptr;  // a TN-column block lies in one 128-row block
  const auto put_products = [&](int s, float sa_v, float sw_v) {
    float* dst = reinterpret_cast<float*>(smem + (s % FT_S) * FT_STAGE + FT_A + FT_B);
    dst[wave * 64 + lane] = sa_v * sw_v;
  };

  const uint8_t* arow = a.a + size_t(row0) * K;
  const uint8_t* wcol = a.w + size_t(col0) * K;
  const auto issue = [&](int s) {
    const uint32_t st = lds0 + uint32_t((s % FT_S) * FT_STAGE);
#pragma unroll
    for (int i = 0; i < 4; ++i) dma16(arow + s * 128, aoff[i], st + uint32_t(wave * 4 + i) * 1024);
#pragma unroll
    for (int i = 0; i < T::BL; ++i) dma16(wcol + s * 128, boff[i], st + uint32_t(FT_A + (wave * T::BL + i) * 1024));
  };
  issue(0);
  if constexpr (F32S)
    if (wave < 2) put_products(0, sarow[0], swcol[0]);
  // Scales, after stage 0 is in flight.
  for (int e = tid; e < KS; e += 256) {
    const size_t i = size_t(col0 / 128) * KS + e;  // a TN-column block lies in one 128-row scale block
    sw_lds[e] = F32S ? a.sw32[i] : e8m0_to_f32(a.sw8[i]);
  }
  if constexpr (!F32S) {
    const int r = min(tid & 127, Mt - 1);
    for (int e = tid; e < 128 * KS; e += 256) sa_lds[e] = a.sa8[size_t(row0 + r) * KS + (e >> 7)];
  }

  // The wave's live 32-row blocks (2 but in a partial last row tile) as a compile-time count: the stage loop then
  // has no branches, and each block's raw MFMA chain starts from a zero operand instead of zeroed registers.
  const int rb_live = __builtin_amdgcn_readfirstlane(min(2, max(0, (Mt - rh * 64 + 31) / 32)));
  v16f_t acc[2][CB];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) acc[rb][cb] = v16f_t{};
  // One stage; NEXT: a stage follows (its ring loads and scale go out here). The last stage is peeled off, so no
  // branch separates the counted scale load from its wait.
  const auto stages = [&](auto rbl) {
    constexpr int RBL = decltype(rbl)::value;
    const auto stage = [&](int s, auto next_c) {
      constexpr bool NEXT = decltype(next_c)::value;
      wait_vm<0>();     // this wave's part of stage s (the only stage in flight)
      __syncthreads();  // every wave's part has landed; the other slot (stage s - 1) is free
      // The next stage's sa goes out before its ring loads, as a counted load (every wave: an unconditional load keeps
      // the count exact; waves 2 and 3 read rows they do not use): the wait for it at the end of this stage leaves
      // those 4 + BL loads in flight (loads retire in order).
      uint32_t sa_next = 0u;
      if constexpr (NEXT) {
        if constexpr (F32S) sa_next = vload_u32(sarow + s + 1);
        issue(s + 1);
      }
      const uint8_t* stb = smem + (s % FT_S) * FT_STAGE;
      const float swv = sw_lds[s];
      float asc[2];
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
        asc[rb] = F32S ? 1.0f : e8m0_to_f32(sa_lds[s * 128 + rh * 64 + rb * 32 + l32]);
      v16f_t raw[2][CB];
      if constexpr (F32S) {
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
          for (int cb = 0; cb < CB; ++cb) raw[rb][cb] = v16f_t{};
      }
      // The stage's operand reads, conversions and MFMAs at raised wave priority, so that a wave holding operands
      // issues ahead of the other workgroup's waves still waiting for theirs (M = 4096 step: 172 against 181 us).
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        v4i aq[2][2], bq[CB][2];
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
          const int n = ch * (TN / 2) + cb * 32 + l32;
#pragma unroll
          for (int x = 0; x < 2; ++x)
            bq[cb][x] = *reinterpret_cast<const v4i*>(stb + FT_A + (n * 8 + ((4 * j + 2 * h + x) ^ lds_swz(n))) * 16);
        }
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
          const int r = rh * 64 + rb * 32 + l32;
#pragma unroll
          for (int x = 0; x < 2; ++x)
            aq[rb][x] = *reinterpret_cast<const v4i*>(stb + (r * 8 + ((4 * j + 2 * h + x) ^ lds_swz(r))) * 16);
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          bf16x8 bf[CB];
#pragma unroll
          for (int cb = 0; cb < CB; ++cb)
            bf[cb] = fp8x8_to_bf16(uint32_t(bq[cb][t >> 1][(t & 1) * 2]), uint32_t(bq[cb][t >> 1][(t & 1) * 2 + 1]),
                                   F32S ? 1.0f : swv);
#pragma unroll
          for (int rb = 0; rb < 2; ++rb) {
            if (rb >= RBL) break;
            const bf16x8 af =
                fp8x8_to_bf16(uint32_t(aq[rb][t >> 1][(t & 1) * 2]), uint32_t(aq[rb][t >> 1][(t & 1) * 2 + 1]), asc[rb]);
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) {
              if constexpr (F32S) raw[rb][cb] = mfma32_bf16(af, bf[cb], raw[rb][cb]);
              else acc[rb][cb] = mfma32_bf16(af, bf[cb], acc[rb][cb]);
            }
          }
        }
      }
      __builtin_amdgcn_s_setprio(0);
      if constexpr (F32S) {
        // Value i of a 32 x 32 block sits at row 8 (i / 4) + 4 h + i % 4: rows in runs of 4, one 16-byte read each.
        const float* sas = reinterpret_cast<const float*>(stb + FT_A + FT_B);
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
          if (rb >= RBL) break;
#pragma unroll
          for (int i4 = 0; i4 < 4; ++i4) {
            const float4 f4 = *reinterpret_cast<const float4*>(sas + rh * 64 + rb * 32 + 8 * i4 + 4 * h);
            const float f[4] = {f4.x, f4.y, f4.z, f4.w};
#pragma unroll
            for (int cb = 0; cb < CB; ++cb)
#pragma unroll
              for (int q = 0; q < 4; ++q) acc[rb][cb][4 * i4 + q] += raw[rb][cb][4 * i4 + q] * f[q];
          }
        }
        if constexpr (NEXT) {  // into stage s - 1's slot, now free
          wait_vm<4 + T::BL>();
          vlanded(sa_next);
          if (wave < 2) put_products(s + 1, __uint_as_float(sa_next), sw_lds[s + 1]);
        }
      }
    };
    for (int s = 0; s + 1 < KS; ++s) stage(s, std::true_type{});
    stage(KS - 1, std::false_type{});
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
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
      for (int i = 0; i < 16; ++i)
        sc[(rh * 64 + rb * 32 + 8 * (i / 4) + 4 * h + (i % 4)) * FT_LDC + ch * (TN / 2) + cb * 32 + l32] =
            f32_to_bf16(acc[rb][cb][i]);
  __syncthreads();
  for (int e = tid; e < Mt * (TN / 8); e += 256) {
    const int r = e / (TN / 8), c8 = (e % (TN / 8)) * 8;
    *reinterpret_cast<uint4*>(a.c + size_t(row0 + r) * a.ldc + col0 + c8) =
        *reinterpret_cast<const uint4*>(sc + r * FT_LDC + c8);
  }
}

template <bool F32S, int TN>
void launch_tiled_t(const Fp8GemmArgs& a, hipStream_t st) {
  const size_t lds = FpTile<TN>::lds(a.K, F32S);
  auto* kern = &fp8_tiled_kernel<F32S, TN>;
  UH_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                               int(lds)));
  kern<<<tile_grid(a.N / TN, (a.M + 127) / 128), 256, lds, st>>>(a);
  UH_CHECK_LAUNCH();
}
// 64-column tiles while 128-column ones would leave fewer than 256 workgroups: twice the workgroups on the same
// serial K loop each. 4096 x 4096 step, 128 / 64 columns: M = 384 55.9 / 52.7 us, 512 56.6 / 53.0, 768 57.4 / 55.6,
// 1024 (256 workgroups of 128 columns) 61.0 / 60.1, 2048 96.1 / 112.5. (A 4-slot ring of 64-column stages, three in
// flight, ran 80 us at M = 384-768: not kept.)
bool tiled_narrow(const Fp8GemmArgs& a) { return size_t(a.N / 128) * ((a.M + 127) / 128) < 256; }
template <bool F32S>
void launch_tiled_f(const Fp8GemmArgs& a, hipStream_t st) {
  if (tiled_narrow(a)) launch_tiled_t<F32S, 64>(a, st);
  else launch_tiled_t<F32S, 128>(a, st);
}

}  // namespace

bool fp8_tiled_fits(const Fp8GemmArgs& a) {
  // two workgroups per CU: 80 KB of LDS each
  return a.N % 128 == 0 && a.K % 128 == 0 && a.ldc % 8 == 0 && FpTile<128>::lds(a.K, a.sa32 != nullptr) <= 80 * 1024;
}

void launch_fp8_tiled(const Fp8GemmArgs& a, hipStream_t st) {
  if (a.M <= 0) return;
  if (!fp8_tiled_fits(a)) throw std::runtime_error("fp8 tiled gemm: N % 128, K % 128, ldc % 8");
  if (!a.a || !a.w || !a.c) throw std::runtime_error("fp8 gemm: null operand");
  if (a.sa32) {
    if (!a.sw32) throw std::runtime_error("fp8 gemm: scales");
    launch_tiled_f<true>(a, st);
  } else {
    if (!a.sa8 || !a.sw8) throw std::runtime_error("fp8 gemm: scales");
    launch_tiled_f<false>(a, st);
  }
}

}  // namespace unholy::kernels
