// Fused producers of the fp8 activations that the GEMVs / GEMMs read:
//   rmsnorm_quant_slices  rmsnorm of rows (ref_elem.hip:62-77) and act_quant_fp8 (block 128) of its bf16 output in
//                         one launch (the reference's elem_fast.hip:52-88, 115-122), over (row, slice) workgroups so
//                         that a decode step's few rows spread over the chip;
//   quant_remote_tokens   act_quant_fp8 (block 128) of the rows x[u2t[u]] for u below a device-side count
//                         (moe_dispatch.hip:280-306): the compact fp8 form of the tokens whose experts run elsewhere.
//
// rmsnorm's sum of squares follows the reference's order exactly: 256 threads, thread t summing values t, t + 256,
// ... (fused multiply-add, as the device compiles `ss += v * v`), a 32-lane xor butterfly per 32-thread group, then
// the same butterfly over the 8 group sums (block_sum, dev.hip.hpp:154-180, written for 32-lane waves). Here the
// 32-lane groups are the halves of a 64-lane wave and the shuffles' offsets stay below 32. The reciprocal square root
// is 1 / sqrt in IEEE single (each correctly rounded: hipcc's default for device division and sqrt) where the
// reference's rsqrtf is the hardware approximation; the CPU oracle computes the same, so the two agree bit for bit,
// and the reference's outputs are within a bf16 ulp of them.
#include <algorithm>
#include <stdexcept>

#include "common.hpp"
#include "numerics.hpp"
#include "unholy/kernels/elem_fast.hpp"
#include "unholy/kernels/moe_dispatch.hpp"

namespace unholy::kernels {

using namespace uh;

namespace {

constexpr int RQ_NT = 256;

// The row's sum of squares, every thread receiving it (red: 8 floats of LDS).
__device__ __forceinline__ float row_sumsq(const bf16* xr, int dim, float* red) {
  const int tid = threadIdx.x;
  float ss = 0.0f;
  for (int i = tid; i < dim; i += RQ_NT) {
    const float v = bf16_to_f32(xr[i]);
    ss = fmaf(v, v, ss);
  }
  for (int o = 16; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
  if ((tid & 31) == 0) red[tid >> 5] = ss;
  __syncthreads();
  float v = (tid & 31) < RQ_NT / 32 ? red[tid & 31] : 0.0f;
  for (int o = 16; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Workgroup (row, slice): the row's scale, then `per` outputs (a multiple of 256) from column blockIdx.y * per; with q,
// each 128-block's amax gives its e8m0 scale and codes, act_quant_fp8's arithmetic.
// VEC (16-byte aligned rows and weights): the row is first copied to LDS with 16-byte loads, the sum of squares read
// back from there in the order above, and the outputs made 8 per thread (16 threads per 128-block, its amax a DPP row
// max, 16-byte y and 8-byte code stores, no barriers). Otherwise one value per thread per 256-chunk from global
// memory, a 128-block's amax over waves 0-1 / 2-3 through LDS. The same values either way.
template <bool VEC>
__global__ __launch_bounds__(RQ_NT) void rmsnorm_quant_kernel(const bf16* __restrict__ x, int ldx,
                                                              const bf16* __restrict__ w, bf16* __restrict__ y, int ldy,
                                                              uint8_t* __restrict__ q, uint8_t* __restrict__ qs,
                                                              int dim, float eps, int per) {
  extern __shared__ __align__(16) uint8_t xs_raw[];  // VEC: the row, dim bf16
  __shared__ float red[RQ_NT / 32];
  __shared__ float bmax[RQ_NT / 64];
  const int row = blockIdx.x, tid = threadIdx.x, wave = tid >> 6;
  const bf16* xr = x + size_t(row) * ldx;
  bf16* yr = y + size_t(row) * ldy;
  if constexpr (VEC) {
    bf16* xs = reinterpret_cast<bf16*>(xs_raw);
    for (int i = tid * 8; i < dim; i += RQ_NT * 8)
      *reinterpret_cast<uint4*>(xs + i) = *reinterpret_cast<const uint4*>(xr + i);
    __syncthreads();
    const float r = 1.0f / sqrtf(row_sumsq(xs, dim, red) / float(dim) + eps);
    const int items = per / 8;  // a multiple of 32: whole 16-thread groups
    for (int it = tid; it < items; it += RQ_NT) {
      const int d = blockIdx.y * per + it * 8;
      const uint4 xv = *reinterpret_cast<const uint4*>(xs + d);
      const uint4 wv = *reinterpret_cast<const uint4*>(w + d);
      const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w}, ww[4] = {wv.x, wv.y, wv.z, wv.w};
      float v[8], am = 0.0f;
      uint32_t yo[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint16_t y0 = f32_to_bf16(__uint_as_float(ww[k] << 16) * (__uint_as_float(xw[k] << 16) * r));
        const uint16_t y1 =
            f32_to_bf16(__uint_as_float(ww[k] & 0xffff0000u) * (__uint_as_float(xw[k] & 0xffff0000u) * r));
        yo[k] = uint32_t(y0) | uint32_t(y1) << 16;
        v[2 * k] = bf16_to_f32(y0);
        v[2 * k + 1] = bf16_to_f32(y1);
        am = fmaxf(am, fmaxf(fabsf(v[2 * k]), fabsf(v[2 * k + 1])));
      }
      *reinterpret_cast<uint4*>(yr + d) = make_uint4(yo[0], yo[1], yo[2], yo[3]);
      if (!q) continue;  // uniform
      am = row16_max(am);
      const Fp8Block blk = fp8_block_scale(am);
      uint32_t c0, c1;
      fp8_codes8(v, blk, c0, c1);
      *reinterpret_cast<uint2*>(q + size_t(row) * dim + d) = make_uint2(c0, c1);
      if ((it & 15) == 0) qs[size_t(row) * (dim / 128) + d / 128] = blk.se;
    }
  } else {
    const float r = 1.0f / sqrtf(row_sumsq(xr, dim, red) / float(dim) + eps);
    for (int c0 = blockIdx.y * per; c0 < int(blockIdx.y + 1) * per; c0 += RQ_NT) {
      const int d = c0 + tid;
      const float t = bf16_to_f32(xr[d]) * r;
      const bf16 yv = f32_to_bf16(bf16_to_f32(w[d]) * t);
      yr[d] = yv;
      if (!q) continue;  // uniform
      const float v = bf16_to_f32(yv);
      float a = fabsf(v);
      for (int o = 32; o >= 1; o >>= 1) a = fmaxf(a, __shfl_xor(a, o));  // max is order-free
      if ((tid & 63) == 0) bmax[wave] = a;
      __syncthreads();
      const Fp8Block blk = fp8_block_scale(fmaxf(bmax[wave & ~1], bmax[wave | 1]));
      __syncthreads();  // bmax is rewritten by the next chunk
      q[size_t(row) * dim + d] = fp8_code(v, blk);
      if ((tid & 127) == 0) qs[size_t(row) * (dim / 128) + d / 128] = blk.se;
    }
  }
}

// rmsnorm_slices (elem_fast.hip:20-38): rmsnorm_quant_kernel's scale and outputs, any dim, no quantization; workgroup
// (row, slice of `per` columns), one value per thread.
__global__ __launch_bounds__(RQ_NT) void rmsnorm_slices_kernel(const bf16* __restrict__ x, int ldx,
                                                               const bf16* __restrict__ w, bf16* __restrict__ y, int ldy,
                                                               int dim, float eps, int per) {
  __shared__ float red[RQ_NT / 32];
  const bf16* xr = x + size_t(blockIdx.x) * ldx;
  const float r = 1.0f / sqrtf(row_sumsq(xr, dim, red) / float(dim) + eps);
  bf16* yr = y + size_t(blockIdx.x) * ldy;
  const int d1 = min(dim, int(blockIdx.y + 1) * per);
  for (int d = blockIdx.y * per + threadIdx.x; d < d1; d += RQ_NT)
    yr[d] = f32_to_bf16(bf16_to_f32(w[d]) * (bf16_to_f32(xr[d]) * r));
}

// hc_post_slices (elem_fast.hip:40-47, dev.hip.hpp:185-201): out[t][j][d] = bf16(fma(post[t][j], x[t][d], s_j)),
// s_j = fma chain over i of comb[t][i][j] * res[t][i][d]; every res value of a column is read before any out value of
// it is written, so out may be res.
__global__ __launch_bounds__(RQ_NT) void hc_post_slices_kernel(const bf16* x, const bf16* res,
                                                               const float* __restrict__ post,
                                                               const float* __restrict__ comb, bf16* out, int hc,
                                                               int dim, int per) {
  const int t = blockIdx.x, d1 = min(dim, int(blockIdx.y + 1) * per);
  const float* pt = post + size_t(t) * hc;
  const float* ct = comb + size_t(t) * hc * hc;
  for (int d = blockIdx.y * per + threadIdx.x; d < d1; d += RQ_NT) {
    const float xv = bf16_to_f32(x[size_t(t) * dim + d]);
    float r[4];
    for (int i = 0; i < hc; ++i) r[i] = bf16_to_f32(res[(size_t(t) * hc + i) * dim + d]);
    for (int j = 0; j < hc; ++j) {
      float s = 0.0f;
      for (int i = 0; i < hc; ++i) s = fmaf(ct[i * hc + j], r[i], s);
      out[(size_t(t) * hc + j) * dim + d] = f32_to_bf16(fmaf(pt[j], xv, s));
    }
  }
}

// 8 values per thread, 16 threads per 128-block (16-byte loads, the amax a DPP row max); items over the device-side
// count, in a grid-stride loop whose bound is uniform so every 16-lane group stays whole.
__global__ __launch_bounds__(256) void quant_remote_tokens_kernel(const bf16* __restrict__ x, int dim,
                                                                  const int32_t* __restrict__ u2t,
                                                                  const MoePlan* __restrict__ plan,
                                                                  uint8_t* __restrict__ q, uint8_t* __restrict__ s) {
  const size_t items = size_t(plan->n_remote_tokens) * (dim / 8);
  for (size_t base = size_t(blockIdx.x) * 256; base < items; base += size_t(gridDim.x) * 256)
    quant_token_item(x, dim, u2t, q, s, base + threadIdx.x, items);
}

}  // namespace

int row_slices(int rows, int dim) { return std::clamp(64 / std::max(rows, 1), 1, std::max(1, dim / RQ_NT)); }

bool rmsnorm_quant_slices(const bf16* x, int ldx, const bf16* w, bf16* y, int ldy, uint8_t* q, uint8_t* qs, int rows,
                          int dim, float eps, hipStream_t st) {
  const int sl = row_slices(rows, dim);
  // The reference's applicability (elem_fast.hip:117): out of place, slices of whole 256-value chunks.
  if (x == y || dim <= 0 || dim % sl || (dim / sl) % RQ_NT) return false;
  if (rows <= 0) return true;
  if (!x || !w || !y || (q && !qs)) throw std::runtime_error("rmsnorm_quant_slices: null operand");
  if (ldx < dim || ldy < dim) throw std::runtime_error("rmsnorm_quant_slices: ldx / ldy < dim");
  const dim3 grid{unsigned(rows), unsigned(sl)};
  const auto a16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  if (ldx % 8 == 0 && ldy % 8 == 0 && a16(x) && a16(y) && a16(w) && size_t(dim) * 2 <= 64 * 1024)
    rmsnorm_quant_kernel<true><<<grid, RQ_NT, size_t(dim) * 2, st>>>(x, ldx, w, y, ldy, q, qs, dim, eps, dim / sl);
  else
    rmsnorm_quant_kernel<false><<<grid, RQ_NT, 0, st>>>(x, ldx, w, y, ldy, q, qs, dim, eps, dim / sl);
  UH_CHECK_LAUNCH();
  return true;
}

void rmsnorm_slices(const bf16* x, int ldx, const bf16* w, bf16* y, int ldy, int rows, int dim, float eps,
                    hipStream_t st) {
  if (x == y) throw std::runtime_error("rmsnorm_slices: in place");
  if (rows <= 0) return;
  if (!x || !w || !y || dim <= 0 || ldx < dim || ldy < dim) throw std::runtime_error("rmsnorm_slices: operands");
  const int s = row_slices(rows, dim);
  rmsnorm_slices_kernel<<<dim3(unsigned(rows), unsigned(s)), RQ_NT, 0, st>>>(x, ldx, w, y, ldy, dim, eps,
                                                                              (dim + s - 1) / s);
  UH_CHECK_LAUNCH();
}
void hc_post_slices(const bf16* x, const bf16* res, const float* post, const float* comb, bf16* out, int T, int hc,
                    int dim, hipStream_t st) {
  if (hc > 4) throw std::runtime_error("hc_post_slices: hc > 4");
  if (T <= 0) return;
  if (hc < 1 || dim <= 0 || !x || !res || !post || !comb || !out) throw std::runtime_error("hc_post_slices: operands");
  const int s = row_slices(T, dim);
  hc_post_slices_kernel<<<dim3(unsigned(T), unsigned(s)), RQ_NT, 0, st>>>(x, res, post, comb, out, hc, dim,
                                                                           (dim + s - 1) / s);
  UH_CHECK_LAUNCH();
}

void quant_remote_tokens(const uint16_t* x, int dim, const int32_t* u2t, const MoePlan* plan, uint8_t* q_dst,
                         uint8_t* s_dst, int max_tokens, hipStream_t st) {
  if (max_tokens <= 0) return;
  if (dim <= 0 || dim % 128) throw std::runtime_error("quant_remote_tokens: dim % 128");
  if (!x || !u2t || !plan || !q_dst || !s_dst) throw std::runtime_error("quant_remote_tokens: null operand");
  if (reinterpret_cast<uintptr_t>(x) % 16) throw std::runtime_error("quant_remote_tokens: x not 16-byte aligned");
  const unsigned grid = unsigned(std::min<size_t>(cdiv(size_t(max_tokens) * (dim / 8), 256), 4096));
  quant_remote_tokens_kernel<<<grid, 256, 0, st>>>(x, dim, u2t, plan, q_dst, s_dst);
  UH_CHECK_LAUNCH();
}

}  // namespace unholy::kernels
