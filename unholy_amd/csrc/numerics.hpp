// Device numerics for gfx950 (wave64). Storage types are raw integers: bf16 = uint16_t, fp8 e4m3fn and
// e2m1 codes and e8m0 scale exponents = uint8_t. Every conversion that decides a stored bit is written out
// here so that it rounds exactly as the reference's device helpers (src/kernels/dev.hip.hpp:40-127):
// bf16 RNE with NaN kept quiet, e4m3fn RNE with the subnormal range scaled by 2^9, power-of-two ceil
// scales as e8m0 bytes.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace uh {

using bf16 = uint16_t;

__device__ __forceinline__ float bf16_to_f32(bf16 v) { return __uint_as_float(uint32_t(v) << 16); }

// Round to nearest even; NaN stays a quiet NaN (dev.hip.hpp:43-48), written out: the reference for the check of the
// hardware conversion below.
__device__ __forceinline__ bf16 f32_to_bf16_sw(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return bf16((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return bf16(u >> 16);
}
// The same rounding in one instruction (v_cvt_pk_bf16_f32): identical to f32_to_bf16_sw on all 2^32 inputs, NaNs
// included (bf16_check_encode compares every one).
__device__ __forceinline__ bf16 f32_to_bf16(float f) { return __builtin_bit_cast(bf16, __bf16(f)); }
__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// OCP e4m3fn decode (dev.hip.hpp:59-63).
__device__ __forceinline__ float e4m3_to_f32(uint8_t v) {
  const uint32_t e = (v >> 3) & 0xf, m = v & 7;
  const float a = e == 0 ? float(m) * (1.0f / 512.0f) : __uint_as_float((e + 120u) << 23 | m << 20);
  return (v & 0x80) ? -a : a;
}

// RNE into e4m3fn for |x| <= 448 (dev.hip.hpp:82-94): below 2^-6 the value is scaled by 2^9 (exact) and
// rounded to an integer mantissa; above, the fp32 mantissa is rounded at 3 bits.
__device__ __forceinline__ uint8_t f32_to_e4m3(float x) {
  uint32_t u = __float_as_uint(x);
  const uint32_t sign = (u >> 24) & 0x80u;
  u &= 0x7fffffffu;
  const int e = int(u >> 23) - 127;
  if (e < -6) return uint8_t(sign | uint32_t(rintf(__uint_as_float(u) * 512.0f)));
  u += 0x7ffffu + ((u >> 20) & 1u);
  return uint8_t(sign | ((u >> 23) - 120u) << 3 | ((u >> 20) & 7u));
}

__device__ __forceinline__ float e8m0_to_f32(uint8_t v) { return __uint_as_float(uint32_t(v) << 23); }

__device__ __forceinline__ float e2m1_to_f32(uint32_t nib) {
  const uint32_t m = nib & 7;
  const float mag = m < 4 ? 0.5f * float(m) : (m == 7 ? 6.0f : float(m - 2));
  return (nib & 8) ? -mag : mag;
}

// 2^ceil(log2(v)) of a positive normal v, as an e8m0 byte (dev.hip.hpp:123-127).
__device__ __forceinline__ uint8_t pow2_ceil_e8m0(float v) {
  const uint32_t b = __float_as_uint(v);
  return uint8_t(int((b >> 23) & 0xff) + ((b & 0x7fffff) != 0 ? 1 : 0));
}

// The e8m0 byte of the smallest power-of-two scale sc with amax / sc <= 448, exactly (integer logic, no
// rounding of amax / 448): amax = f * 2^E, f in [1, 2): E - 8 when f <= 1.75 (448 = 1.75 * 2^8), else E - 7.
// Used to recover the fp8 codes of values that are already e4m3 * 2^k (fake-quantized rows): any such scale
// leaves every code exact. amax == 0 gives 127 (codes all zero).
__device__ __forceinline__ uint8_t exact_fp8_scale(float amax) {
  const uint32_t b = __float_as_uint(amax);
  if (b == 0) return 127;
  const int E = int(b >> 23);  // biased
  return uint8_t(E - 8 + ((b & 0x7fffff) > 0x600000u ? 1 : 0));
}

// Wave64 reductions over all 64 lanes (every lane active).
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
// Max over groups of G consecutive lanes (G a power of two <= 64).
template <int G>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int o = G / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Uniform wave64 reductions of 32-bit unsigned values through DPP (pairs, quads, half-rows, rows) and four lane
// reads, instead of a shuffle per level: a few cycles per level rather than an LDS round trip.
template <bool MAX>
__device__ __forceinline__ uint32_t wave_reduce_u32(uint32_t v) {
  const auto op = [](uint32_t a, uint32_t b) { return MAX ? (a > b ? a : b) : (a < b ? a : b); };
  v = op(v, uint32_t(__builtin_amdgcn_update_dpp(int(v), int(v), 0xB1, 0xf, 0xf, false)));   // quad_perm [1,0,3,2]
  v = op(v, uint32_t(__builtin_amdgcn_update_dpp(int(v), int(v), 0x4E, 0xf, 0xf, false)));   // quad_perm [2,3,0,1]
  v = op(v, uint32_t(__builtin_amdgcn_update_dpp(int(v), int(v), 0x141, 0xf, 0xf, false)));  // row_half_mirror
  v = op(v, uint32_t(__builtin_amdgcn_update_dpp(int(v), int(v), 0x140, 0xf, 0xf, false)));  // row_mirror
  const uint32_t r0 = __builtin_amdgcn_readlane(v, 0), r1 = __builtin_amdgcn_readlane(v, 16);
  const uint32_t r2 = __builtin_amdgcn_readlane(v, 32), r3 = __builtin_amdgcn_readlane(v, 48);
  return op(op(r0, r1), op(r2, r3));
}
// Max over each aligned group of 16 lanes (a DPP row), every lane of the group receiving it: two quad
// permutations then rotations by 4 and 8 within the row. All 16 lanes of a group must be active.
template <int CTRL>
__device__ __forceinline__ float dpp_max_step(float x) {
  return fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(x), __float_as_int(x), CTRL, 0xf, 0xf,
                                                             false)));
}
__device__ __forceinline__ float row16_max(float v) {
  v = dpp_max_step<0xB1>(v);   // quad_perm [1,0,3,2]
  v = dpp_max_step<0x4E>(v);   // quad_perm [2,3,0,1]
  v = dpp_max_step<0x124>(v);  // row_ror:4
  return dpp_max_step<0x128>(v);  // row_ror:8
}
// A float's bits mapped so that unsigned order is float order.
__device__ __forceinline__ uint32_t orderable(float f) {
  const uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// The reference's activation fake quantization of one value given its block's amax (ref_elem.hip:32-37):
// amax floored at 1e-4, e8m0 scale 2^ceil(log2(amax / 448)), e4m3 RNE of the clamped quotient.
// inv = 1 / sc exactly (se lies in [105, 247]: the amax floor and the fp32 range keep 2^(127 - se) normal), so
// v * inv is the correctly rounded v / sc, the same value the division gives, without the IEEE division sequence.
struct Fp8Block {
  uint8_t se;
  float sc;
  float inv;
};
__device__ __forceinline__ Fp8Block fp8_block_scale(float amax) {
  const uint8_t se = pow2_ceil_e8m0(fmaxf(amax, 1e-4f) * (1.0f / 448.0f));
  return {se, e8m0_to_f32(se), __uint_as_float(uint32_t(254 - se) << 23)};
}
// e4m3 codes (round to nearest even) of values already in [-448, 448] with the hardware encode v_cvt_pk_fp8_f32:
// on that range it gives exactly the codes of f32_to_e4m3 (fp8_check_encode compares every fp32 value of it).
// Byte i of e4m3x4 is value i.
__device__ __forceinline__ uint8_t e4m3_hw(float x) {
  return uint8_t(__builtin_amdgcn_cvt_pk_fp8_f32(x, 0.0f, 0, false));
}
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d) {
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return uint32_t(__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true));
}
__device__ __forceinline__ float clamp448(float v) { return fminf(fmaxf(v, -448.0f), 448.0f); }
// Any positive fp32 scale (the fp32-scale activation format): a true division.
__device__ __forceinline__ uint8_t fp8_code(float v, float sc) { return e4m3_hw(clamp448(v / sc)); }
__device__ __forceinline__ uint8_t fp8_code(float v, const Fp8Block& b) { return e4m3_hw(clamp448(v * b.inv)); }
// The codes of 8 values of one block, lowest byte first.
__device__ __forceinline__ void fp8_codes8(const float (&v)[8], const Fp8Block& b, uint32_t& lo, uint32_t& hi) {
  lo = e4m3x4(clamp448(v[0] * b.inv), clamp448(v[1] * b.inv), clamp448(v[2] * b.inv), clamp448(v[3] * b.inv));
  hi = e4m3x4(clamp448(v[4] * b.inv), clamp448(v[5] * b.inv), clamp448(v[6] * b.inv), clamp448(v[7] * b.inv));
}
__device__ __forceinline__ void fp8_codes8(const float (&v)[8], float sc, uint32_t& lo, uint32_t& hi) {
  lo = e4m3x4(clamp448(v[0] / sc), clamp448(v[1] / sc), clamp448(v[2] / sc), clamp448(v[3] / sc));
  hi = e4m3x4(clamp448(v[4] / sc), clamp448(v[5] / sc), clamp448(v[6] / sc), clamp448(v[7] / sc));
}

// act_quant_fp8 (block 128) of compact token rows: item `it` of items = U * dim / 8 is 8 values of row x[u2t[u]]
// (16-byte load), 16 consecutive items one 128-block (amax a DPP row max). Every lane of a 16-lane group must call
// it, items past the end included (they clamp to the last item for the max and store nothing).
__device__ __forceinline__ void quant_token_item(const uint16_t* __restrict__ x, int dim,
                                                 const int32_t* __restrict__ u2t, uint8_t* __restrict__ q,
                                                 uint8_t* __restrict__ s, size_t it, size_t items) {
  const size_t ic = it < items ? it : items - 1;
  const int per_row = dim / 8;
  const int u = int(ic / per_row), rem = int(ic % per_row), b = rem >> 4, l = rem & 15;
  const uint4 raw = *reinterpret_cast<const uint4*>(x + size_t(u2t[u]) * dim + b * 128 + 8 * l);
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
  if (it >= items) return;
  const Fp8Block blk = fp8_block_scale(am);
  uint32_t c0, c1;
  fp8_codes8(v, blk, c0, c1);
  *reinterpret_cast<uint2*>(q + size_t(u) * dim + b * 128 + 8 * l) = make_uint2(c0, c1);
  if (l == 0) s[size_t(u) * (dim / 128) + b] = blk.se;
}

// e^x from IEEE operations only (fma, mul, rint; no hardware approximation), so that the kernels and the CPU oracle
// compute the same bits everywhere e^x decides a stored value (the SwiGLU's silu, the softmax and sigmoid routers'
// weights). Cody-Waite reduction x = n ln2 + r with ln2 split into a 16-significant-bit high part (n ln2_hi is
// exact for |n| <= 150) and the rest, |r| <= ln2 / 2; e^r by its degree-7 Taylor polynomial in Horner form with
// fused multiply-adds (truncation below 2^-27 relative); results down to the subnormal range are one rounding of
// p 2^n (the oracle applies 2^n as two exact power-of-two factors, here v_ldexp_f32 rounds p 2^n once: the same
// value). Within 2 ulp of e^x (tests/test_oracle.py).
// Branch-free: the polynomial path runs for every x, on x clamped into [-103.972084, 88.7228394] (unchanged inside
// it), and the results past the cut-offs are selected at the end, so a wave of mixed inputs takes no divergent
// branch.
__device__ __forceinline__ float exp_f32(float x) {
#pragma clang fp contract(off)  // every rounding as written (no multiply-add fused into the caller's add)
  const float xc = __builtin_amdgcn_fmed3f(x, -103.972084f, 88.7228394f);  // NaN: replaced below
  const float n = rintf(xc * 1.44269504f);
  float r = __builtin_fmaf(-n, 0.693145751953125f, xc);
  r = __builtin_fmaf(-n, 1.42860677e-06f, r);
  float p = 1.0f / 5040.0f;
  p = __builtin_fmaf(p, r, 1.0f / 720.0f);
  p = __builtin_fmaf(p, r, 1.0f / 120.0f);
  p = __builtin_fmaf(p, r, 1.0f / 24.0f);
  p = __builtin_fmaf(p, r, 1.0f / 6.0f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  float e = __builtin_amdgcn_ldexpf(p, int(n));
  asm volatile("" : "+v"(e));  // computed on every path: the compiler would otherwise branch around it
  // x >= 88.7228394: +inf, or x itself (quieted) when x is NaN
  return !(x < 88.7228394f) ? x + __builtin_inff() : x < -103.972084f ? 0.0f : e;
}

// SwiGLU with the clamp and optional routing weight (ref_moe.hip:62-74): x = silu(min(g, l)) * clamp(u, +-l), then
// w * x; limit <= 0 turns the clamp off. e^x is exp_f32.
__device__ __forceinline__ float swiglu_value(float g, float u, float w, bool has_w, float limit) {
#pragma clang fp contract(off)
  if (limit > 0.0f) {
    u = fminf(fmaxf(u, -limit), limit);
    g = fminf(g, limit);
  }
  float x = (g / (1.0f + exp_f32(-g))) * u;
  if (has_w) x = w * x;
  return x;
}

}  // namespace uh
