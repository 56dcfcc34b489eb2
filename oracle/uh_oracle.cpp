// CPU oracle for the quantized MoE expert path and the fp8 block-scaled dense GEMM.
//
// TEST INFRASTRUCTURE ONLY. Nothing in the product (unholy_amd/, include/) links, loads or calls this file;
// it is the checker for the HIP kernels (tests/), the smoke check (__graft_entry__.smoke) and the timed
// CPU baseline leg of bench.py. It restates, on the host and in plain C++, the arithmetic of the
// reference's device reference kernels, in the same operation order, so that its fp32 results are the
// reference's bit for bit:
//
//   numerics            src/kernels/dev.hip.hpp:40-127 (device codecs), src/core/half.hpp:68-96 (host twins)
//   act_quant_fp8       src/kernels/ref_elem.hip:18-41 (e8m0 scales); tools/ref/oracle/kernel.py:43-55
//                       (scale_fmt=None: fp32 scales amax/448)
//   fake_quant_fp4      src/kernels/ref_elem.hip:43-59 (e2m1 per block, amax floor 6 * 2^-126), round_e2m1
//                       dev.hip.hpp:107-119
//   gemm_a8w4(_tiled)   src/kernels/ref_gemm.hip:15-67 (K-block partial sums), :77-99, :138-155, :180-188
//   gemm_w8a8           src/kernels/ref_gemm.hip:130-137, :175-178; fp32-scale form: gemm_wmma.hip:89-100
//                       (raw per-128 chain folded with acc += raw * (sa * sw))
//   gemm_grouped_fp8w   src/kernels/ref_gemm.hip:111-125, :198-202 with gemm_ref_kernel :18-67 at G = K (one
//                       K-block: a single fp32 fmaf chain over k in order, scale 1): "mgk,grk->mgr"
//   rmsnorm (+ quant)   src/kernels/ref_elem.hip:62-77 (rmsnorm_kernel, 256 threads), dev.hip.hpp:154-180
//                       (block_sum: a wave32 xor butterfly per warp, then the same butterfly over the warp sums);
//                       elem_fast.hip:52-88 (rmsnorm_quant_slices: act_quant_fp8 per 128 of the bf16 output).
//                       The sum of squares as the device compiles `ss += v * v` (contracted: fma). One deviation:
//                       1 / sqrt in IEEE single (sqrt, then divide, each correctly rounded) where the reference's
//                       rsqrtf is the hardware approximation, which no CPU restatement reproduces
//   swiglu              src/kernels/ref_moe.hip:62-74
//   route (DSV4)        src/kernels/ref_moe.hip:14-60
//   route (GLM sigmoid) src/kernels/moe_dispatch.hip:308-356
//   moe_combine         src/kernels/ref_moe.hip:90-99
//   dispatch order      src/model/forward_ref.hip:1302-1328 (host path: experts ascending, resident first,
//                       tokens ascending within an expert, each token's picks sorted by expert id)
//   tile lists          src/kernels/moe_dispatch.hip:39-79 (<= tile_rows rows per tile, experts in order)
//   tile-major layout   src/model/expert_pack.cpp:146-166 (repack_matrix / unrepack_matrix)
//   expert composition  src/model/forward_ref.hip:268-304 (act_quant -> gemm_a8w4 w1, w3 -> swiglu ->
//                       act_quant -> gemm_a8w4 w2), then moe_combine
//
// The softmax top-k router is the synthetic workload's router (not in the reference): selection by logit,
// descending, ties to the lower expert id (softmax is monotone); weight_i = exp(l_i - m) / sum over the
// picks in selection order of exp(l_j - m), m = the first pick's logit: the renormalised softmax.
//
// The *_f64 functions are the fp64 oracle: the same quantized operands, products and sums in double,
// no rounding before the output (only summation order separates them from an exact result).
//
// Build: oracle/Makefile (g++ -O2 -ffp-contract=off: every fp32 operation rounds where written).
#include <algorithm>
#include <array>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

namespace {

inline float u2f(uint32_t u) {
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}
inline uint32_t f2u(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return u;
}

// dev.hip.hpp:40
inline float bf16_to_f32(uint16_t v) { return u2f(uint32_t(v) << 16); }
// dev.hip.hpp:43-48: round to nearest even, NaN kept as a quiet NaN.
inline uint16_t f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}
inline float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }
// dev.hip.hpp:59-63 (OCP e4m3fn; the device decode has no NaN case, the quantizer never emits 0x7f/0xff).
inline float e4m3_to_f32(uint8_t v) {
  const uint32_t e = (v >> 3) & 0xf, m = v & 7;
  const float a = e == 0 ? float(m) * (1.0f / 512.0f) : u2f((e + 120u) << 23 | m << 20);
  return (v & 0x80) ? -a : a;
}
// dev.hip.hpp:82-94: RNE into e4m3fn, |x| <= 448 (callers clamp).
inline uint8_t f32_to_e4m3(float x) {
  uint32_t u = f2u(x);
  const uint8_t sign = uint8_t((u >> 24) & 0x80);
  u &= 0x7fffffffu;
  const int e = int(u >> 23) - 127;
  if (e < -6) {
    const float r = std::nearbyint(u2f(u) * 512.0f);  // default rounding mode: nearest even
    return uint8_t(sign | uint8_t(r));
  }
  u += 0x7ffffu + ((u >> 20) & 1u);
  const uint32_t ee = (u >> 23) - 127 + 7, man = (u >> 20) & 7;
  return uint8_t(sign | uint8_t(ee << 3 | man));
}
// dev.hip.hpp:96
inline float e8m0_to_f32(uint8_t v) { return u2f(uint32_t(v) << 23); }
// dev.hip.hpp:99-104; half.hpp:90-94
inline float e2m1_to_f32(uint32_t nib) {
  static constexpr float kLut[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
  const float m = kLut[nib & 7];
  return (nib & 8) ? -m : m;
}
// dev.hip.hpp:123-127
inline uint8_t pow2_ceil_e8m0(float v) {
  const uint32_t b = f2u(v);
  const int e = int((b >> 23) & 0xff) - 127 + ((b & 0x7fffff) != 0 ? 1 : 0);
  return uint8_t(e + 127);
}

// e2m1 rounding of a scaled value, to nearest with ties to the even code (dev.hip.hpp:107-119: the midpoints 0.25,
// 1.25, 2.5 and 5 go down, 0.75, 1.75 and 3.5 go up).
inline float round_e2m1(float x) {
  const float a = std::fabs(x);
  float r;
  if (a <= 0.25f) r = 0.0f;
  else if (a < 0.75f) r = 0.5f;
  else if (a <= 1.25f) r = 1.0f;
  else if (a < 1.75f) r = 1.5f;
  else if (a <= 2.5f) r = 2.0f;
  else if (a < 3.5f) r = 3.0f;
  else if (a <= 5.0f) r = 4.0f;
  else r = 6.0f;
  return x < 0 ? -r : r;
}

// e^x as the library computes it (IEEE operations only, so both sides produce the same bits; the reference's device
// expf is an ocml routine no CPU restatement reproduces): Cody-Waite reduction with ln2 split into a 16-bit-exact
// high part and the rest, the degree-7 Taylor polynomial of e^r in Horner form with fused multiply-adds, and 2^n as
// two exact power-of-two factors.
inline float pow2_f32(int e) { return u2f(uint32_t(e + 127) << 23); }
inline float exp_f32(float x) {
  if (!(x < 88.7228394f)) return x != x ? x : INFINITY;
  if (x < -103.972084f) return 0.0f;
  const float n = std::rint(x * 1.44269504f);
  float r = std::fma(-n, 0.693145751953125f, x);
  r = std::fma(-n, 1.42860677e-06f, r);
  float p = 1.0f / 5040.0f;
  p = std::fma(p, r, 1.0f / 720.0f);
  p = std::fma(p, r, 1.0f / 120.0f);
  p = std::fma(p, r, 1.0f / 24.0f);
  p = std::fma(p, r, 1.0f / 6.0f);
  p = std::fma(p, r, 0.5f);
  p = std::fma(p, r, 1.0f);
  p = std::fma(p, r, 1.0f);
  const int ni = int(n), h = ni / 2;
  return (p * pow2_f32(h)) * pow2_f32(ni - h);
}

// Runs f(i) for i in [0, n) on up to nthreads threads (contiguous ranges).
template <class F>
void parallel_for(int n, int nthreads, F f) {
  nthreads = std::max(1, std::min(nthreads, n));
  if (nthreads == 1) {
    for (int i = 0; i < n; ++i) f(i);
    return;
  }
  std::vector<std::thread> th;
  for (int t = 0; t < nthreads; ++t)
    th.emplace_back([&, t] {
      const int a = int(int64_t(n) * t / nthreads), b = int(int64_t(n) * (t + 1) / nthreads);
      for (int i = a; i < b; ++i) f(i);
    });
  for (auto& x : th) x.join();
}

// Code byte of (row n, input k) of a packed e2m1 matrix: row-major [N, K/2] or the tile-major layout.
inline uint8_t e2m1_byte(const uint8_t* w, int N, int K, int n, int k, bool tiled) {
  if (!tiled) return w[size_t(n) * (K / 2) + k / 2];
  const size_t chunk = size_t(k / 64) * (N / 16) + n / 16;  // ref_gemm.hip:95-96
  return w[chunk * 512 + (n % 16) * 32 + (k % 64) / 2];
}
inline float e2m1_at(const uint8_t* w, int N, int K, int n, int k, bool tiled) {
  const uint8_t b = e2m1_byte(w, N, K, n, k, tiled);
  return e2m1_to_f32((k & 1) ? (b >> 4) : (b & 0xf));
}
inline uint8_t e2m1_scale(const uint8_t* s, int N, int K, int n, int kb32, bool tiled) {
  if (!tiled) return s[size_t(n) * (K / 32) + kb32];
  const size_t chunk = size_t(kb32 / 2) * (N / 16) + n / 16;  // ref_gemm.hip:152-153
  return s[chunk * 32 + (n % 16) * 2 + kb32 % 2];
}

}  // namespace

extern "C" {

// ---- scalar codecs (exported for the known-answer tests) ----------------------------------------------
float or_bf16_to_f32(uint16_t v) { return bf16_to_f32(v); }
uint16_t or_f32_to_bf16(float f) { return f32_to_bf16(f); }
float or_e4m3_to_f32(uint8_t v) { return e4m3_to_f32(v); }
uint8_t or_f32_to_e4m3(float x) { return f32_to_e4m3(x); }
float or_e8m0_to_f32(uint8_t v) { return e8m0_to_f32(v); }
float or_e2m1_to_f32(uint32_t nib) { return e2m1_to_f32(nib); }
void or_exp_f32_array(const float* x, float* y, size_t n) {
  for (size_t i = 0; i < n; ++i) y[i] = exp_f32(x[i]);
}
uint8_t or_pow2_ceil_e8m0(float v) { return pow2_ceil_e8m0(v); }

void or_f32_to_bf16_array(const float* x, uint16_t* y, size_t n) {
  for (size_t i = 0; i < n; ++i) y[i] = f32_to_bf16(x[i]);
}
void or_f32_to_e4m3_array(const float* x, uint8_t* y, size_t n) {
  for (size_t i = 0; i < n; ++i) y[i] = f32_to_e4m3(x[i]);
}

// ---- activation quantization (ref_elem.hip:18-41) -------------------------------------------------------
// x bf16 [rows, ldx] -> q e4m3 [rows, cols], s e8m0 [rows, cols / block].
void or_act_quant_fp8(const uint16_t* x, int ldx, uint8_t* q, uint8_t* s, int rows, int cols, int block) {
  const int nb = cols / block;
  for (int r = 0; r < rows; ++r)
    for (int b = 0; b < nb; ++b) {
      const uint16_t* xr = x + size_t(r) * ldx + size_t(b) * block;
      float amax = 0.0f;
      for (int i = 0; i < block; ++i) amax = std::fmax(amax, std::fabs(bf16_to_f32(xr[i])));
      amax = std::fmax(amax, 1e-4f);
      const uint8_t se = pow2_ceil_e8m0(amax * (1.0f / 448.0f));
      const float sc = e8m0_to_f32(se);
      for (int i = 0; i < block; ++i)
        q[size_t(r) * cols + size_t(b) * block + i] =
            f32_to_e4m3(std::fmin(std::fmax(bf16_to_f32(xr[i]) / sc, -448.0f), 448.0f));
      s[size_t(r) * nb + b] = se;
    }
}
// In-place e2m1 fake quantization per block (ref_elem.hip:43-59): amax floored at 6 * 2^-126, sc = 2^ceil(log2(amax /
// 6)), x = bf16(e2m1(clamp(x / sc, +-6)) * sc).
void or_fake_quant_fp4(uint16_t* x, int ldx, int rows, int cols, int block) {
  const int nb = cols / block;
  for (int r = 0; r < rows; ++r)
    for (int b = 0; b < nb; ++b) {
      uint16_t* xr = x + size_t(r) * ldx + size_t(b) * block;
      float amax = 0.0f;
      for (int i = 0; i < block; ++i) amax = std::fmax(amax, std::fabs(bf16_to_f32(xr[i])));
      amax = std::fmax(amax, 6.0f * 1.1754943508222875e-38f);
      const float sc = e8m0_to_f32(pow2_ceil_e8m0(amax * (1.0f / 6.0f)));
      for (int i = 0; i < block; ++i)
        xr[i] = f32_to_bf16(round_e2m1(std::fmin(std::fmax(bf16_to_f32(xr[i]) / sc, -6.0f), 6.0f)) * sc);
    }
}
// In-place fake quantization: x = bf16(e4m3(x / sc) * sc) per block (ref_elem.hip:37).
void or_fake_quant_fp8(uint16_t* x, int ldx, int rows, int cols, int block) {
  const int nb = cols / block;
  std::vector<uint8_t> q(static_cast<size_t>(block));
  for (int r = 0; r < rows; ++r)
    for (int b = 0; b < nb; ++b) {
      uint8_t se;
      uint16_t* xr = x + size_t(r) * ldx + size_t(b) * block;
      or_act_quant_fp8(xr, block, q.data(), &se, 1, block, block);
      const float sc = e8m0_to_f32(se);
      for (int i = 0; i < block; ++i) xr[i] = f32_to_bf16(e4m3_to_f32(q[size_t(i)]) * sc);
    }
}
// kernel.py act_quant with scale_fmt=None: s = max(amax, 1e-4) * fp32(1/448), q = e4m3(clamp(x / s)).
void or_act_quant_fp8_f32s(const uint16_t* x, int ldx, uint8_t* q, float* s, int rows, int cols, int block) {
  const int nb = cols / block;
  for (int r = 0; r < rows; ++r)
    for (int b = 0; b < nb; ++b) {
      const uint16_t* xr = x + size_t(r) * ldx + size_t(b) * block;
      float amax = 0.0f;
      for (int i = 0; i < block; ++i) amax = std::fmax(amax, std::fabs(bf16_to_f32(xr[i])));
      amax = std::fmax(amax, 1e-4f);
      const float sc = amax * (1.0f / 448.0f);
      for (int i = 0; i < block; ++i)
        q[size_t(r) * cols + size_t(b) * block + i] =
            f32_to_e4m3(std::fmin(std::fmax(bf16_to_f32(xr[i]) / sc, -448.0f), 448.0f));
      s[size_t(r) * nb + b] = sc;
    }
}

// ---- tile-major MXFP4 layout (expert_pack.cpp:146-166) -----------------------------------------------------
void or_repack(const uint8_t* w, const uint8_t* s, uint8_t* tw, uint8_t* ts, int N, int K) {
  const size_t rb = size_t(K) / 2, nb = size_t(K) / 64, rs = size_t(K) / 32, n16 = size_t(N) / 16;
  for (size_t r = 0; r < size_t(N); ++r) {
    for (size_t j = 0; j < nb; ++j)
      std::memcpy(tw + ((j * n16 + r / 16) * 512 + (r % 16) * 32), w + r * rb + j * 32, 32);
    for (size_t b = 0; b < rs; ++b) ts[((b / 2) * n16 + r / 16) * 32 + (r % 16) * 2 + b % 2] = s[r * rs + b];
  }
}
void or_unrepack(const uint8_t* tw, const uint8_t* ts, uint8_t* w, uint8_t* s, int N, int K) {
  const size_t rb = size_t(K) / 2, nb = size_t(K) / 64, rs = size_t(K) / 32, n16 = size_t(N) / 16;
  for (size_t r = 0; r < size_t(N); ++r) {
    for (size_t j = 0; j < nb; ++j)
      std::memcpy(w + r * rb + j * 32, tw + ((j * n16 + r / 16) * 512 + (r % 16) * 32), 32);
    for (size_t b = 0; b < rs; ++b) s[r * rs + b] = ts[((b / 2) * n16 + r / 16) * 32 + (r % 16) * 2 + b % 2];
  }
}
// Dequantized weight matrix [N, K] as fp32 (exact: e2m1 * 2^(s - 127)).
void or_mx_dequant(const uint8_t* w, const uint8_t* s, float* out, int N, int K, int tiled) {
  for (int n = 0; n < N; ++n)
    for (int k = 0; k < K; ++k)
      out[size_t(n) * K + k] = e2m1_at(w, N, K, n, k, tiled) * e8m0_to_f32(e2m1_scale(s, N, K, n, k / 32, tiled));
}

// ---- GEMMs, C[M,N] = A[M,K] W[N,K]^T ---------------------------------------------------------------------------
// gemm_a8w4: per 32-block partial sums (k ascending, fmaf) scaled by sa[m][k/128] * sw[n][k/32] and added in
// block order (ref_gemm.hip:26-58 with G = 32). c: bf16 (c16) or fp32 (c32) or both.
void or_gemm_a8w4(const uint8_t* a, const uint8_t* sa, const uint8_t* w, const uint8_t* sw, uint16_t* c16, float* c32,
                  int ldc, int M, int N, int K, int tiled, int nthreads) {
  // Every output is the fma chain of ref_gemm.hip:54-63 in its order. The activations are decoded once; NB adjacent
  // columns are decoded one 64-input slab at a time (a tile that stays in L1), and their chains run side by side
  // (the same chains, interleaved for the CPU's pipelines).
  constexpr int NB = 32;
  static const auto lut = [] {
    std::array<std::array<float, 2>, 256> t{};
    for (int b = 0; b < 256; ++b) t[size_t(b)] = {e2m1_to_f32(uint32_t(b) & 0xf), e2m1_to_f32(uint32_t(b) >> 4)};
    return t;
  }();
  std::vector<float> af(size_t(M) * K), asc(size_t(M) * (K / 128));
  for (size_t i = 0; i < af.size(); ++i) af[i] = e4m3_to_f32(a[i]);
  for (size_t i = 0; i < asc.size(); ++i) asc[i] = e8m0_to_f32(sa[i]);
  parallel_for((N + NB - 1) / NB, nthreads, [&](int nb) {
    const int n0 = nb * NB, cols = std::min(NB, N - n0);
    std::vector<float> part(size_t(M) * NB, 0.0f), acc(size_t(M) * NB, 0.0f);
    alignas(64) float wt[64][NB];
    float wsc[2][NB];
    for (int kt = 0; kt < K / 64; ++kt) {
      for (int j = 0; j < NB; ++j) {
        const int n = n0 + std::min(j, cols - 1);
        const uint8_t* src = &w[tiled ? (size_t(kt) * (N / 16) + n / 16) * 512 + (n % 16) * 32
                                      : size_t(n) * (K / 2) + size_t(kt) * 32];
        for (int i = 0; i < 32; ++i) {
          wt[2 * i][j] = lut[src[i]][0];
          wt[2 * i + 1][j] = lut[src[i]][1];
        }
        for (int h = 0; h < 2; ++h) wsc[h][j] = e8m0_to_f32(e2m1_scale(sw, N, K, n, 2 * kt + h, tiled != 0));
      }
      for (int m = 0; m < M; ++m) {
        const float* ar = &af[size_t(m) * K + size_t(kt) * 64];
        float* pm = &part[size_t(m) * NB];
        float* am = &acc[size_t(m) * NB];
        for (int h = 0; h < 2; ++h) {
          for (int k = 32 * h; k < 32 * h + 32; ++k) {
            const float ak = ar[k];
            for (int j = 0; j < NB; ++j) pm[j] = std::fma(ak, wt[k][j], pm[j]);
          }
          const float sam = asc[size_t(m) * (K / 128) + kt / 2];
          for (int j = 0; j < NB; ++j) {
            am[j] += pm[j] * (sam * wsc[h][j]);
            pm[j] = 0.0f;
          }
        }
      }
    }
    for (int m = 0; m < M; ++m)
      for (int j = 0; j < cols; ++j) {
        const float v = acc[size_t(m) * NB + j];
        if (c16) c16[size_t(m) * ldc + n0 + j] = f32_to_bf16(v);
        if (c32) c32[size_t(m) * ldc + n0 + j] = v;
      }
  });
}
void or_gemm_a8w4_f64(const uint8_t* a, const uint8_t* sa, const uint8_t* w, const uint8_t* sw, double* c, int ldc,
                      int M, int N, int K, int tiled, int nthreads) {
  parallel_for(N, nthreads, [&](int n) {
    for (int m = 0; m < M; ++m) {
      double acc = 0.0;
      for (int k = 0; k < K; ++k)
        acc += double(e4m3_to_f32(a[size_t(m) * K + k])) * double(e2m1_at(w, N, K, n, k, tiled != 0)) *
               double(e8m0_to_f32(sa[size_t(m) * (K / 128) + k / 128])) *
               double(e8m0_to_f32(e2m1_scale(sw, N, K, n, k / 32, tiled != 0)));
      c[size_t(m) * ldc + n] = acc;
    }
  });
}

// gemm_w8a8: per 128-block partial sums scaled by sa[m][kb] * sw[n/128][kb] (e8m0; ref_gemm.hip:130-137, G = 128).
// sa32 / sw32 non-null: fp32 scales instead (kernel.py fp8_gemm with scale_fmt=None; gemm_wmma.hip:89-100 fold).
void or_gemm_w8a8(const uint8_t* a, const uint8_t* sa, const float* sa32, const uint8_t* w, const uint8_t* sw,
                  const float* sw32, uint16_t* c16, float* c32, int ldc, int M, int N, int K, int nthreads) {
  // The chains of ref_gemm.hip:130-137 in their order; activations decoded once, each column's weights once, NB
  // adjacent columns' chains side by side.
  constexpr int NB = 32;
  const int kbs = K / 128;
  std::vector<float> af(size_t(M) * K);
  for (size_t i = 0; i < af.size(); ++i) af[i] = e4m3_to_f32(a[i]);
  parallel_for((N + NB - 1) / NB, nthreads, [&](int nb) {
    const int n0 = nb * NB, cols = std::min(NB, N - n0);
    std::vector<float> wv(size_t(K) * NB, 0.0f);  // [k][column]
    for (int j = 0; j < cols; ++j)
      for (int k = 0; k < K; ++k) wv[size_t(k) * NB + j] = e4m3_to_f32(w[size_t(n0 + j) * K + k]);
    for (int m = 0; m < M; ++m) {
      const float* ar = &af[size_t(m) * K];
      float acc[NB] = {};
      for (int kb = 0; kb < kbs; ++kb) {
        float part[NB] = {};
        for (int k = kb * 128; k < kb * 128 + 128; ++k) {
          const float ak = ar[k];
          const float* wk = &wv[size_t(k) * NB];
          for (int j = 0; j < NB; ++j) part[j] = std::fma(ak, wk[j], part[j]);
        }
        for (int j = 0; j < cols; ++j) {
          const int n = n0 + j;
          const float sc = sa32 ? sa32[size_t(m) * kbs + kb] * sw32[size_t(n / 128) * kbs + kb]
                                : e8m0_to_f32(sa[size_t(m) * kbs + kb]) * e8m0_to_f32(sw[size_t(n / 128) * kbs + kb]);
          acc[j] += part[j] * sc;
        }
      }
      for (int j = 0; j < cols; ++j) {
        if (c16) c16[size_t(m) * ldc + n0 + j] = f32_to_bf16(acc[j]);
        if (c32) c32[size_t(m) * ldc + n0 + j] = acc[j];
      }
    }
  });
}
void or_gemm_w8a8_f64(const uint8_t* a, const uint8_t* sa, const float* sa32, const uint8_t* w, const uint8_t* sw,
                      const float* sw32, double* c, int ldc, int M, int N, int K, int nthreads) {
  const int kbs = K / 128;
  parallel_for(N, nthreads, [&](int n) {
    for (int m = 0; m < M; ++m) {
      double acc = 0.0;
      for (int kb = 0; kb < kbs; ++kb) {
        double part = 0.0;
        for (int k = kb * 128; k < kb * 128 + 128; ++k)
          part += double(e4m3_to_f32(a[size_t(m) * K + k])) * double(e4m3_to_f32(w[size_t(n) * K + k]));
        const double sc = sa32 ? double(sa32[size_t(m) * kbs + kb]) * double(sw32[size_t(n / 128) * kbs + kb])
                                : double(e8m0_to_f32(sa[size_t(m) * kbs + kb])) *
                                      double(e8m0_to_f32(sw[size_t(n / 128) * kbs + kb]));
        acc += part * sc;
      }
      c[size_t(m) * ldc + n] = acc;
    }
  });
}

// gemm_grouped_fp8w: c[m][g][r] = bf16(fmaf chain over k of bf16 a[m][g][k] * (e4m3 w[g R + r][k] * e8m0
// sw[(g R + r) / 128][k / 128])), the weight product exact in fp32 (ref_gemm.hip:116-125; gemm_ref_kernel at G = K).
void or_gemm_grouped_fp8w(const uint16_t* a, const uint8_t* w, const uint8_t* sw, uint16_t* c16, float* c32, int M,
                          int G, int R, int K, int nthreads) {
  const int kbs = K / 128;
  parallel_for(G * R, nthreads, [&](int n) {
    const int g = n / R;
    std::vector<float> wv(static_cast<size_t>(K));
    for (int k = 0; k < K; ++k)
      wv[size_t(k)] = e4m3_to_f32(w[size_t(n) * K + k]) * e8m0_to_f32(sw[size_t(n / 128) * kbs + k / 128]);
    for (int m = 0; m < M; ++m) {
      const uint16_t* am = a + (size_t(m) * G + g) * K;
      float acc = 0.0f;
      for (int k = 0; k < K; ++k) acc = std::fma(bf16_to_f32(am[k]), wv[size_t(k)], acc);
      if (c16) c16[size_t(m) * G * R + n] = f32_to_bf16(acc);
      if (c32) c32[size_t(m) * G * R + n] = acc;
    }
  });
}
void or_gemm_grouped_fp8w_f64(const uint16_t* a, const uint8_t* w, const uint8_t* sw, double* c, int M, int G, int R,
                              int K, int nthreads) {
  const int kbs = K / 128;
  parallel_for(G * R, nthreads, [&](int n) {
    const int g = n / R;
    for (int m = 0; m < M; ++m) {
      const uint16_t* am = a + (size_t(m) * G + g) * K;
      double acc = 0.0;
      for (int k = 0; k < K; ++k)
        acc += double(bf16_to_f32(am[k])) * double(e4m3_to_f32(w[size_t(n) * K + k])) *
               double(e8m0_to_f32(sw[size_t(n / 128) * kbs + k / 128]));
      c[size_t(m) * G * R + n] = acc;
    }
  });
}

// rmsnorm of rows [rows, dim] in the reference's order, then (q set) act_quant_fp8 (block 128) of the bf16 output.
void or_rmsnorm_quant(const uint16_t* x, int ldx, const uint16_t* w, uint16_t* y, int ldy, uint8_t* q, uint8_t* qs,
                      int rows, int dim, float eps) {
  constexpr int NT = 256;
  for (int r = 0; r < rows; ++r) {
    const uint16_t* xr = x + size_t(r) * ldx;
    float part[NT];
    for (int t = 0; t < NT; ++t) {
      float ss = 0.0f;
      for (int i = t; i < dim; i += NT) {
        const float v = bf16_to_f32(xr[i]);
        ss = std::fma(v, v, ss);
      }
      part[t] = ss;
    }
    // block_sum: within each 32-thread warp v += v[lane ^ o] for o = 16, 8, 4, 2, 1 (every lane ends with the same
    // value), then warp 0 repeats it over the 8 warp sums (lanes 8-31 hold zero: the first two steps add zero).
    const auto butterfly = [](float* v) {
      for (int o = 16; o >= 1; o >>= 1) {
        float nv[32];
        for (int l = 0; l < 32; ++l) nv[l] = v[l] + v[l ^ o];
        std::memcpy(v, nv, sizeof(nv));
      }
    };
    float red[32] = {};
    for (int wv = 0; wv < NT / 32; ++wv) {
      float v[32];
      std::memcpy(v, part + wv * 32, sizeof(v));
      butterfly(v);
      red[wv] = v[0];
    }
    butterfly(red);
    const float rinv = 1.0f / std::sqrt(red[0] / float(dim) + eps);
    uint16_t* yr = y + size_t(r) * ldy;
    for (int i = 0; i < dim; ++i) {
      const float t = bf16_to_f32(xr[i]) * rinv;
      yr[i] = f32_to_bf16(bf16_to_f32(w[i]) * t);
    }
  }
  if (q) or_act_quant_fp8(y, ldy, q, qs, rows, dim, 128);
}

// ---- SwiGLU (ref_moe.hip:62-74) -----------------------------------------------------------------------------------
void or_swiglu(const uint16_t* gate, const uint16_t* up, const float* w, uint16_t* h, int rows, int dim, float limit) {
  for (size_t i = 0; i < size_t(rows) * dim; ++i) {
    float g = bf16_to_f32(gate[i]), u = bf16_to_f32(up[i]);
    if (limit > 0.0f) {
      u = std::fmin(std::fmax(u, -limit), limit);
      g = std::fmin(g, limit);
    }
    float x = (g / (1.0f + exp_f32(-g))) * u;
    if (w) x = w[i / size_t(dim)] * x;
    h[i] = f32_to_bf16(x);
  }
}

// ---- routers --------------------------------------------------------------------------------------------------------
// DSV4 route (ref_moe.hip:14-60): sqrt(softplus(logit)) + bias selects (hash layers: tid2eid[ids[t]]), ties to
// the lower id; weights = score / sum(score) * route_scale in selection order. bias_vl: image tokens' bias.
void or_route_ds(const float* logits, const float* bias0, const int32_t* tid2eid0, const int32_t* ids, int32_t* sel,
                 float* weights, int T, int E, int K, float route_scale, const float* bias_vl, int vocab) {
  for (int t = 0; t < T; ++t) {
    const bool image = bias_vl && ids[t] >= vocab;
    const float* bias = image ? bias_vl : bias0;
    const int32_t* tid2eid = image ? nullptr : tid2eid0;
    const float* lg = logits + size_t(t) * E;
    auto score = [&](int e) {
      const float x = lg[e];
      const float sp = x > 20.0f ? x : std::log1p(std::exp(x));
      return std::sqrt(sp);
    };
    int chosen[8];
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
          const float v = score(e) + bias[e];
          if (best < 0 || v > bv) best = e, bv = v;
        }
        chosen[k] = best;
      }
    }
    float w[8], sum = 0.0f;
    for (int k = 0; k < K; ++k) {
      w[k] = score(chosen[k]);
      sum += w[k];
    }
    for (int k = 0; k < K; ++k) {
      sel[size_t(t) * K + k] = chosen[k];
      weights[size_t(t) * K + k] = (w[k] / sum) * route_scale;
    }
  }
}
// GLM route (moe_dispatch.hip:308-356): sigmoid(logit) + bias selects, picks reported in ascending expert id,
// weights = sigmoid / (sum + 1e-20) * route_scale (sum in ascending-id order).
void or_route_glm(const float* logits, const float* bias, int32_t* sel, float* wt, int T, int E, int K,
                  float route_scale) {
  for (int t = 0; t < T; ++t) {
    const float* lr = logits + size_t(t) * E;
    std::vector<float> sv(static_cast<size_t>(E));
    for (int e = 0; e < E; ++e) sv[size_t(e)] = 1.0f / (1.0f + exp_f32(-lr[e])) + bias[e];
    int chosen[8];
    for (int k = 0; k < K; ++k) {
      int bi = -1;
      for (int e = 0; e < E; ++e)
        if (sv[size_t(e)] != -INFINITY && (bi < 0 || sv[size_t(e)] > sv[size_t(bi)])) bi = e;
      chosen[k] = bi;
      sv[size_t(bi)] = -INFINITY;
    }
    std::sort(chosen, chosen + K);
    float s[8], sum = 0.0f;
    for (int k = 0; k < K; ++k) {
      s[k] = 1.0f / (1.0f + exp_f32(-lr[chosen[k]]));
      sum += s[k];
    }
    for (int k = 0; k < K; ++k) {
      sel[size_t(t) * K + k] = chosen[k];
      wt[size_t(t) * K + k] = s[k] / (sum + 1e-20f) * route_scale;
    }
  }
}
// Softmax top-K, renormalised over the picks (the synthetic workload's router; see the file header).
void or_route_softmax(const float* logits, int32_t* sel, float* wt, int T, int E, int K) {
  for (int t = 0; t < T; ++t) {
    const float* lr = logits + size_t(t) * E;
    int chosen[8];
    for (int k = 0; k < K; ++k) {
      int bi = -1;
      for (int e = 0; e < E; ++e) {
        bool used = false;
        for (int j = 0; j < k; ++j) used |= chosen[j] == e;
        if (used) continue;
        if (bi < 0 || lr[e] > lr[bi]) bi = e;
      }
      chosen[k] = bi;
    }
    const float m = lr[chosen[0]];
    float ev[8], sum = 0.0f;
    for (int k = 0; k < K; ++k) {
      ev[k] = exp_f32(lr[chosen[k]] - m);
      sum += ev[k];
    }
    for (int k = 0; k < K; ++k) {
      sel[size_t(t) * K + k] = chosen[k];
      wt[size_t(t) * K + k] = ev[k] / sum;
    }
  }
}

// ---- dispatch (forward_ref.hip:1302-1328 order; moe_dispatch.hip:39-79 tiles) -------------------------------------
// resident: null = all resident. tiles: int32 triples {expert, row0, rows}. plan: {P, remote0, n_local_tiles,
// n_remote_tiles, n_remote_tokens}. Returns the local tile count (not capped).
int or_dispatch(const int32_t* sel, const float* wt, int T, int K, int E, const uint8_t* resident, int tile_rows,
                int32_t* count, int32_t* off, int32_t* eidx, float* ewt, int32_t* row_expert, int32_t* pidx,
                int32_t* tiles, int max_tiles, int32_t* remote_tiles, int32_t* plan) {
  std::fill(count, count + E, 0);
  for (int i = 0; i < T * K; ++i) ++count[sel[i]];
  int next = 0, remote0 = 0;
  for (int pass = 0; pass < 2; ++pass) {
    if (pass == 1) remote0 = next;
    for (int e = 0; e < E; ++e)
      if ((resident ? resident[e] != 0 : true) == (pass == 0)) {
        off[e] = next;
        next += count[e];
      }
  }
  std::vector<int> fill(off, off + E);
  for (int t = 0; t < T; ++t) {
    std::vector<std::pair<int32_t, float>> picks;
    for (int j = 0; j < K; ++j) picks.push_back({sel[size_t(t) * K + j], wt[size_t(t) * K + j]});
    std::stable_sort(picks.begin(), picks.end(), [](auto& a, auto& b) { return a.first < b.first; });
    for (int j = 0; j < K; ++j) {
      const int e = picks[size_t(j)].first;
      const int p = fill[size_t(e)]++;
      eidx[p] = t;
      ewt[p] = picks[size_t(j)].second;
      row_expert[p] = e;
      pidx[size_t(t) * K + j] = p;
    }
  }
  int nl = 0, nr = 0;
  for (int e = 0; e < E; ++e) {
    const bool loc = resident ? resident[e] != 0 : true;
    for (int i = 0; i < count[e]; i += tile_rows) {
      int32_t* dst = loc ? tiles : remote_tiles;
      int& n = loc ? nl : nr;
      if (dst && n < max_tiles) {
        dst[3 * n] = e;
        dst[3 * n + 1] = off[e] + i;
        dst[3 * n + 2] = std::min(tile_rows, count[e] - i);
      }
      ++n;
    }
  }
  if (plan) {
    plan[0] = T * K;
    plan[1] = remote0;
    plan[2] = std::min(nl, max_tiles);
    plan[3] = std::min(nr, max_tiles);
    plan[4] = 0;
  }
  return nl;
}

// ---- combine (ref_moe.hip:90-99) -------------------------------------------------------------------------------------
void or_moe_combine(const uint16_t* pair_out, const int32_t* pidx, const uint16_t* shared, uint16_t* out, int T, int K,
                    int dim) {
  for (int t = 0; t < T; ++t)
    for (int d = 0; d < dim; ++d) {
      float acc = 0.0f;
      for (int j = 0; j < K; ++j) acc += bf16_to_f32(pair_out[size_t(pidx[size_t(t) * K + j]) * dim + d]);
      acc += shared ? bf16_to_f32(shared[size_t(t) * dim + d]) : 0.0f;
      out[size_t(t) * dim + d] = f32_to_bf16(acc);
    }
}

// ---- remote experts: compact tokens and partial combines (moe_dispatch.hip:149-278) ---------------------------------
// remote_tokens (moe_dispatch.hip:149-203): token t has a remote pair when one of its pair rows is >= remote0; those
// tokens, in token order, get compact indices u. tok2u [T] (-1: none), u2t [U], p2u[p] = tok2u[eidx[p]] for
// p in [remote0, P), u2p [U, K] (optional) = token u's j-th pair row if remote, else -1. Returns U.
int or_remote_tokens(const int32_t* pidx, const int32_t* eidx, int T, int K, int remote0, int P, int32_t* tok2u,
                     int32_t* u2t, int32_t* p2u, int32_t* u2p) {
  int U = 0;
  for (int t = 0; t < T; ++t) {
    bool f = false;
    for (int j = 0; j < K; ++j) f = f || pidx[size_t(t) * K + j] >= remote0;
    tok2u[t] = f ? U : -1;
    if (!f) continue;
    u2t[U] = t;
    if (u2p)
      for (int j = 0; j < K; ++j) {
        const int p = pidx[size_t(t) * K + j];
        u2p[size_t(U) * K + j] = p >= remote0 ? p : -1;
      }
    ++U;
  }
  for (int p = remote0; p < P; ++p) p2u[p] = tok2u[eidx[p]];
  return U;
}

// remote_combine (moe_dispatch.hip:206-229): dst[u] = bf16(sum over j of pair_out[u2p[u][j]] for u2p >= 0), fp32
// adds from 0 in j order.
void or_remote_combine(const uint16_t* pair_out, const int32_t* u2p, int U, int K, int dim, uint16_t* dst) {
  for (int u = 0; u < U; ++u)
    for (int d = 0; d < dim; ++d) {
      float acc = 0.0f;
      for (int j = 0; j < K; ++j) {
        const int p = u2p[size_t(u) * K + j];
        if (p >= 0) acc += bf16_to_f32(pair_out[size_t(p) * dim + d]);
      }
      dst[size_t(u) * dim + d] = f32_to_bf16(acc);
    }
}

// moe_combine_partial / _link (moe_dispatch.hip:243-278): out[t] = bf16(local pair rows (p < remote0, j order) +
// remote row tok2u[t] (if any) + shared[t]), fp32 adds from 0. remote: the remote rows (pair_out + remote0 * dim for
// moe_combine_partial, remote_combine's dst for the link form). shared null: no term. hc_x non-null: the mHC post-mix
// (dev.hip.hpp:185-201) of the combined value o into the streams hc_x [T][hc][dim] in place:
// x[t][j][d] = bf16(fma(post[t][j], o, s_j)), s_j = fma chain over i of comb[t][i][j] * x[t][i][d] (old values).
void or_moe_combine_partial(const uint16_t* pair_out, const int32_t* pidx, int remote0, const int32_t* tok2u,
                            const uint16_t* remote, const uint16_t* shared, uint16_t* out, int T, int K, int dim,
                            uint16_t* hc_x, const float* post, const float* comb, int hc) {
  for (int t = 0; t < T; ++t)
    for (int d = 0; d < dim; ++d) {
      float acc = 0.0f;
      for (int j = 0; j < K; ++j) {
        const int p = pidx[size_t(t) * K + j];
        if (p < remote0) acc += bf16_to_f32(pair_out[size_t(p) * dim + d]);
      }
      const int u = tok2u[t];
      if (u >= 0) acc += bf16_to_f32(remote[size_t(u) * dim + d]);
      if (shared) acc += bf16_to_f32(shared[size_t(t) * dim + d]);
      const uint16_t o = f32_to_bf16(acc);
      out[size_t(t) * dim + d] = o;
      if (!hc_x) continue;
      float r[4];
      for (int i = 0; i < hc; ++i) r[i] = bf16_to_f32(hc_x[(size_t(t) * hc + i) * dim + d]);
      for (int j = 0; j < hc; ++j) {
        float s = 0.0f;
        for (int i = 0; i < hc; ++i) s = std::fma(comb[(size_t(t) * hc + i) * hc + j], r[i], s);
        hc_x[(size_t(t) * hc + j) * dim + d] = f32_to_bf16(std::fma(post[size_t(t) * hc + j], bf16_to_f32(o), s));
      }
    }
}

// hc_post (ref_elem.hip hc_post, dev.hip.hpp:185-201): out[t][j][d] = bf16(fma(post[t][j], x[t][d], s_j)), s_j an
// fma chain from 0 over i of comb[t][i][j] * res[t][i][d]. out may be res (a column's res values are read first).
void or_hc_post(const uint16_t* x, const uint16_t* res, const float* post, const float* comb, uint16_t* out, int T,
                int hc, int dim) {
  for (int t = 0; t < T; ++t)
    for (int d = 0; d < dim; ++d) {
      float r[4];
      for (int i = 0; i < hc; ++i) r[i] = bf16_to_f32(res[(size_t(t) * hc + i) * dim + d]);
      for (int j = 0; j < hc; ++j) {
        float s = 0.0f;
        for (int i = 0; i < hc; ++i) s = std::fma(comb[(size_t(t) * hc + i) * hc + j], r[i], s);
        out[(size_t(t) * hc + j) * dim + d] =
            f32_to_bf16(std::fma(post[size_t(t) * hc + j], bf16_to_f32(x[size_t(t) * dim + d]), s));
      }
    }
}

// ---- the routed-expert FFN (forward_ref.hip:268-304 per expert, then moe_combine) ------------------------------------
// x bf16 [T, D]; sel / wt [T, K]; per-expert tables of code and scale pointers for w1, w3 ([I, D]) and w2
// ([D, I]), raw or tile-major (tiled). Experts with a null w1 code pointer are skipped (their pair rows are
// left as pair_out holds them on entry). pair_out bf16 [T*K, D] (the host dispatch order); out bf16 [T, D].
// experts_subset (optional, n_subset entries): only those experts are computed (the timed CPU sample).
void or_moe_forward(const uint16_t* x, const int32_t* sel, const float* wt, int T, int K, int E, int D, int I,
                    const uint8_t* const* w1, const uint8_t* const* s1, const uint8_t* const* w3,
                    const uint8_t* const* s3, const uint8_t* const* w2, const uint8_t* const* s2, int tiled,
                    float limit, uint16_t* pair_out, uint16_t* out, int nthreads, const int32_t* experts_subset,
                    int n_subset, uint8_t* hq_out, uint8_t* hs_out) {
  const int P = T * K;
  std::vector<int32_t> count(static_cast<size_t>(E)), off(static_cast<size_t>(E)), eidx(static_cast<size_t>(P)), row_expert(static_cast<size_t>(P)), pidx(static_cast<size_t>(P));
  std::vector<float> ewt(static_cast<size_t>(P));
  or_dispatch(sel, wt, T, K, E, nullptr, 128, count.data(), off.data(), eidx.data(), ewt.data(), row_expert.data(),
              pidx.data(), nullptr, 0, nullptr, nullptr);
  std::vector<int> experts;
  if (experts_subset)
    experts.assign(experts_subset, experts_subset + n_subset);
  else
    for (int e = 0; e < E; ++e) experts.push_back(e);
  // Experts with rows in parallel (each has its own rows); when there are fewer of them than threads, the GEMMs of
  // each expert split their output columns over the rest.
  {
    std::vector<int> live;
    for (int e : experts)
      if (count[size_t(e)] > 0 && w1[e]) live.push_back(e);
    experts.swap(live);
  }
  const int inner = std::max(1, nthreads / std::max(1, int(experts.size())));
  parallel_for(int(experts.size()), nthreads, [&](int ie) {
    const int e = experts[size_t(ie)];
    const int cnt = count[size_t(e)], r0 = off[size_t(e)];
    if (cnt == 0 || !w1[e]) return;
    std::vector<uint16_t> in(size_t(cnt) * D), h1(size_t(cnt) * I), h3(size_t(cnt) * I), hh(size_t(cnt) * I);
    for (int r = 0; r < cnt; ++r)
      std::memcpy(&in[size_t(r) * D], x + size_t(eidx[size_t(r0 + r)]) * D, size_t(D) * 2);
    std::vector<uint8_t> q(size_t(cnt) * std::max(D, I)), qs(size_t(cnt) * (std::max(D, I) / 128));
    or_act_quant_fp8(in.data(), D, q.data(), qs.data(), cnt, D, 128);
    or_gemm_a8w4(q.data(), qs.data(), w1[e], s1[e], h1.data(), nullptr, I, cnt, I, D, tiled, inner);
    or_gemm_a8w4(q.data(), qs.data(), w3[e], s3[e], h3.data(), nullptr, I, cnt, I, D, tiled, inner);
    or_swiglu(h1.data(), h3.data(), &ewt[size_t(r0)], hh.data(), cnt, I, limit);
    or_act_quant_fp8(hh.data(), I, q.data(), qs.data(), cnt, I, 128);
    if (hq_out) std::memcpy(hq_out + size_t(r0) * I, q.data(), size_t(cnt) * I);  // h's codes and scales, optional
    if (hs_out) std::memcpy(hs_out + size_t(r0) * (I / 128), qs.data(), size_t(cnt) * (I / 128));
    or_gemm_a8w4(q.data(), qs.data(), w2[e], s2[e], pair_out + size_t(r0) * D, nullptr, D, cnt, D, I, tiled, inner);
  });
  if (out) or_moe_combine(pair_out, pidx.data(), nullptr, out, T, K, D);
}

}  // extern "C"
