// The C ABI (include/unholy_amd.h): exception-to-status wrappers over the C++ entry points, device memory and
// stream helpers for hosts without a HIP binding (the Python package binds this library with ctypes), the
// synthetic-data generator and the one-call routed-expert FFN.
#include <fcntl.h>
#include <unistd.h>

#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>

#include "common.hpp"
#include "numerics.hpp"
#include "unholy/kernels/elem_fast.hpp"
#include "unholy/model/expert_pack.hpp"
#include "unholy/kernels/gemm_wmma.hpp"
#include "unholy/kernels/gemv.hpp"
#include "unholy/kernels/moe_dispatch.hpp"
#include "unholy/kernels/mx_moe.hpp"
#include "unholy/kernels/ref.hpp"
#include "unholy_amd.h"
#include "mx_internal.hpp"

namespace k = unholy::kernels;
using uh::bf16;

namespace {

thread_local std::string g_err;

template <class F>
int guard(F&& f) {
  try {
    f();
    return 0;
  } catch (const std::exception& e) {
    g_err = e.what();
  } catch (...) {
    g_err = "unknown error";
  }
  return -1;
}

inline hipStream_t S(void* s) { return static_cast<hipStream_t>(s); }
inline const k::Exl3Tile* T3(const int32_t* p) { return reinterpret_cast<const k::Exl3Tile*>(p); }

__global__ void fill_random_kernel(uint8_t* dst, size_t n, uint64_t seed, uint32_t lo, uint32_t span) {
  for (size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x; i < (n + 7) / 8; i += size_t(gridDim.x) * blockDim.x) {
    uint64_t z = seed + 0x9e3779b97f4a7c15ull * (i + 1);  // splitmix64
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    z ^= z >> 31;
    for (int b = 0; b < 8 && i * 8 + b < n; ++b) dst[i * 8 + b] = uint8_t(lo + uint32_t((z >> (8 * b)) & 0xff) % span);
  }
}

// Weight quantization for the dense fp8 workload: a block per 128 x 128 tile, amax over the tile.
__global__ __launch_bounds__(256) void quant_weight_kernel(const float* w, uint8_t* q, float* s, int N, int K) {
  __shared__ float red[4];
  const int bn = blockIdx.y, bk = blockIdx.x, kb = K / 128;
  float am = 0.0f;
  for (int i = threadIdx.x; i < 128 * 128; i += 256) {
    const int r = bn * 128 + i / 128, c = bk * 128 + i % 128;
    if (r < N) am = fmaxf(am, fabsf(w[size_t(r) * K + c]));
  }
  am = uh::wave_max(am);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = am;
  __syncthreads();
  am = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float sc = fmaxf(am, 1e-4f) * (1.0f / 448.0f);
  for (int i = threadIdx.x; i < 128 * 128; i += 256) {
    const int r = bn * 128 + i / 128, c = bk * 128 + i % 128;
    if (r < N) q[size_t(r) * K + c] = uh::fp8_code(w[size_t(r) * K + c], sc);
  }
  if (threadIdx.x == 0) s[size_t(bn) * kb + bk] = sc;
}

__global__ void exp_f32_kernel(const float* x, float* y, size_t n) {
  for (size_t i = blockIdx.x * size_t(blockDim.x) + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x)
    y[i] = uh::exp_f32(x[i]);
}

// UH_PREFILL_FP8=1: the prefill forward feeds the GEMMs e4m3 codes + scales (mx_grouped_gemm_q) instead of bf16
// rows (comparison runs; both are bit-identical). The block-scaled speed mode (mx_gemm_set_exact(0)) always takes
// the e4m3 codes, the operands of its MFMA.
static bool prefill_fp8() {
  static const bool on = [] {
    const char* e = std::getenv("UH_PREFILL_FP8");
    return e && e[0] == '1';
  }();
  return on;
}

// Workspace carve-up of uh_mx_moe_forward.
struct MoeWs {
  int32_t *count, *off, *fill, *plan, *tiles, *eidx, *row_expert, *pidx, *sel;
  float *ewt, *wt;
  uint8_t *xq, *xs, *hq, *hs;
  bf16 *xa, *hh;  // prefill: fake-quantized token rows [T, D] (in xq's bytes) and SwiGLU rows [P, I]
  bf16* h;  // raw SwiGLU rows [P, I] (T <= 64 path); shares xq's bytes (P * D >= P * I * 2), which only prefill uses
  bf16* pair_out;
  size_t bytes;
  int max_tiles, tile_rows;
};
MoeWs carve(char* base, int T, int K, int E, int D, int I) {
  MoeWs w{};
  const size_t P = size_t(T) * K;
  w.tile_rows = T <= 64 ? 16 : k::kExl3TileRows;
  w.max_tiles = int(std::min<size_t>(P, size_t(E) + P / size_t(w.tile_rows) + 1));
  size_t o = 0;
  auto take = [&](size_t bytes) {
    char* p = base ? base + o : nullptr;
    o += (bytes + 255) / 256 * 256;
    return p;
  };
  w.count = reinterpret_cast<int32_t*>(take(size_t(E) * 4));
  w.off = reinterpret_cast<int32_t*>(take(size_t(E) * 4));
  w.fill = reinterpret_cast<int32_t*>(take(size_t(E) * 4));
  w.plan = reinterpret_cast<int32_t*>(take(sizeof(k::MoePlan)));
  w.tiles = reinterpret_cast<int32_t*>(take(size_t(w.max_tiles) * sizeof(k::Exl3Tile)));
  w.eidx = reinterpret_cast<int32_t*>(take(P * 4));
  w.row_expert = reinterpret_cast<int32_t*>(take(P * 4));
  w.pidx = reinterpret_cast<int32_t*>(take(P * 4));
  w.sel = reinterpret_cast<int32_t*>(take(P * 4));
  w.ewt = reinterpret_cast<float*>(take(P * 4));
  w.wt = reinterpret_cast<float*>(take(P * 4));
  w.xq = reinterpret_cast<uint8_t*>(take(P * D));
  w.h = reinterpret_cast<bf16*>(w.xq);
  if (size_t(D) < size_t(I) * 2) w.h = reinterpret_cast<bf16*>(take(P * I * 2));
  w.xs = reinterpret_cast<uint8_t*>(take(P * (D / 128)));
  w.hq = reinterpret_cast<uint8_t*>(take(P * I));
  w.hs = reinterpret_cast<uint8_t*>(take(P * (I / 128)));
  w.xa = reinterpret_cast<bf16*>(w.xq);  // T * D * 2 <= P * D
  w.hh = T > 64 ? reinterpret_cast<bf16*>(take(P * I * 2)) : nullptr;
  w.pair_out = reinterpret_cast<bf16*>(take(P * D * 2));
  w.bytes = o;
  return w;
}

// The no-allocation forward's workspace: one fixed array per device, for callers that cannot allocate (code under
// graph capture, serving loops). Each GPU holds its own copy until the process ends; host code reaches it only
// through the address hipGetSymbolAddress returns on that device (the array's name is a host-side stand-in there).
constexpr size_t kScratchBytes = size_t(8) << 20;
__device__ __align__(256) uint8_t scratch[kScratchBytes];
constexpr int kMaxDevices = 64;
std::once_flag g_scratch_once[kMaxDevices];
void* g_scratch_ptr[kMaxDevices];

// The current device's scratch address, looked up once per device with that device current.
void* scratch_ptr() {
  int dev = 0;
  UH_CHECK(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) throw std::runtime_error("uh_mx_moe_forward_noalloc: device id out of range");
  std::call_once(g_scratch_once[dev], [dev] {
    void* p = nullptr;
    UH_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) throw std::runtime_error("uh_mx_moe_forward_noalloc: no scratch address on device " + std::to_string(dev));
    g_scratch_ptr[dev] = p;
  });
  if (!g_scratch_ptr[dev]) throw std::runtime_error("uh_mx_moe_forward_noalloc: scratch lookup failed earlier");
  return g_scratch_ptr[dev];
}

}  // namespace

extern "C" {

const char* uh_last_error(void) { return g_err.c_str(); }
int uh_version(void) { return 1; }
int uh_device_count(int* n) {
  return guard([&] { UH_CHECK(hipGetDeviceCount(n)); });
}
int uh_set_device(int dev) {
  return guard([&] { UH_CHECK(hipSetDevice(dev)); });
}
int uh_device_name(char* buf, int len) {
  return guard([&] {
    int dev = 0;
    UH_CHECK(hipGetDevice(&dev));
    hipDeviceProp_t p{};
    UH_CHECK(hipGetDeviceProperties(&p, dev));
    std::snprintf(buf, size_t(len), "%s (%s, %d CUs)", p.name, p.gcnArchName, p.multiProcessorCount);
  });
}
int uh_malloc(void** p, size_t bytes) {
  return guard([&] { UH_CHECK(hipMalloc(p, bytes ? bytes : 1)); });
}
int uh_free(void* p) {
  return guard([&] { UH_CHECK(hipFree(p)); });
}
int uh_memcpy_h2d(void* dst, const void* src, size_t bytes) {
  return guard([&] { UH_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice)); });
}
int uh_memcpy_d2h(void* dst, const void* src, size_t bytes) {
  return guard([&] { UH_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost)); });
}
int uh_memcpy_d2d(void* dst, const void* src, size_t bytes, void* st) {
  return guard([&] { UH_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, S(st))); });
}
int uh_memset(void* dst, int value, size_t bytes, void* st) {
  return guard([&] { UH_CHECK(hipMemsetAsync(dst, value, bytes, S(st))); });
}
int uh_synchronize(void) {
  return guard([&] { UH_CHECK(hipDeviceSynchronize()); });
}
int uh_stream_create(void** st) {
  return guard([&] {
    hipStream_t s;
    UH_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *st = s;
  });
}
int uh_stream_destroy(void* st) {
  return guard([&] { UH_CHECK(hipStreamDestroy(S(st))); });
}
int uh_stream_synchronize(void* st) {
  return guard([&] { UH_CHECK(hipStreamSynchronize(S(st))); });
}
int uh_event_create(void** ev) {
  return guard([&] {
    hipEvent_t e;
    UH_CHECK(hipEventCreate(&e));
    *ev = e;
  });
}
int uh_event_destroy(void* ev) {
  return guard([&] { UH_CHECK(hipEventDestroy(static_cast<hipEvent_t>(ev))); });
}
int uh_event_record(void* ev, void* st) {
  return guard([&] { UH_CHECK(hipEventRecord(static_cast<hipEvent_t>(ev), S(st))); });
}
int uh_event_synchronize(void* ev) {
  return guard([&] { UH_CHECK(hipEventSynchronize(static_cast<hipEvent_t>(ev))); });
}
int uh_event_elapsed_ms(float* ms, void* a, void* b) {
  return guard([&] { UH_CHECK(hipEventElapsedTime(ms, static_cast<hipEvent_t>(a), static_cast<hipEvent_t>(b))); });
}
int uh_graph_capture_begin(void* st) {
  return guard([&] {
    if (!st) throw std::runtime_error("uh_graph_capture_begin: capture needs a created stream");
    UH_CHECK(hipStreamBeginCapture(static_cast<hipStream_t>(st), hipStreamCaptureModeThreadLocal));
  });
}
int uh_graph_capture_end(void* st, void** exec) {
  return guard([&] {
    hipGraph_t g = nullptr;
    UH_CHECK(hipStreamEndCapture(static_cast<hipStream_t>(st), &g));
    hipGraphExec_t e = nullptr;
    const hipError_t r = hipGraphInstantiate(&e, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    UH_CHECK(r);
    *exec = e;
  });
}
int uh_graph_launch(void* exec, void* st) {
  return guard([&] { UH_CHECK(hipGraphLaunch(static_cast<hipGraphExec_t>(exec), static_cast<hipStream_t>(st))); });
}
int uh_graph_destroy(void* exec) {
  return guard([&] { UH_CHECK(hipGraphExecDestroy(static_cast<hipGraphExec_t>(exec))); });
}
int uh_fill_random_bytes(void* dst, size_t n, uint64_t seed, uint32_t lo, uint32_t hi, void* st) {
  return guard([&] {
    if (hi < lo || hi > 255) throw std::runtime_error("uh_fill_random_bytes: need lo <= hi <= 255");
    if (!n) return;
    const unsigned grid = unsigned(std::min<size_t>(uh::cdiv((n + 7) / 8, 256), 65536));
    fill_random_kernel<<<grid, 256, 0, S(st)>>>(static_cast<uint8_t*>(dst), n, seed, lo, hi - lo + 1);
    UH_CHECK_LAUNCH();
  });
}

int uh_mx_repack(uint8_t* w, uint8_t* s, int N, int K, uint8_t* tmp, void* st) {
  return guard([&] { k::mx_repack(w, s, N, K, tmp, S(st)); });
}
int uh_mx_repack_to(const uint8_t* w, const uint8_t* s, uint8_t* tw, uint8_t* ts, int N, int K, void* st) {
  return guard([&] { k::mx_repack_to(w, s, tw, ts, N, K, S(st)); });
}
int uh_mx_xform_in(const uint16_t* x, int ldx, const int32_t* row_expert, const uint8_t* const* s_tab, uint16_t* xa,
                   int P, int K, void* st, const int32_t* x_rows) {
  return guard([&] { k::mx_xform_in(x, ldx, row_expert, s_tab, xa, P, K, S(st), x_rows); });
}
int uh_mx_xform_in_fp8(const uint16_t* x, int ldx, const int32_t* row_expert, const uint8_t* const* s_tab,
                       uint8_t* q, uint8_t* qs, int P, int K, void* st, const int32_t* x_rows) {
  return guard([&] { k::mx_xform_in_fp8(x, ldx, row_expert, s_tab, q, qs, P, K, S(st), x_rows); });
}
int uh_mx_swiglu(const uint16_t* g, const uint16_t* u, const float* w, const int32_t* row_expert,
                 const uint8_t* const* s_tab, uint16_t* hh, int P, int I, float limit, void* st) {
  return guard([&] { k::mx_swiglu(g, u, w, row_expert, s_tab, hh, P, I, limit, S(st)); });
}
int uh_check_fp8_encode(unsigned long long* bad, unsigned long long* total) {
  return guard([&] { *bad = k::fp8_check_encode(total); });
}

int uh_check_bf16_encode(unsigned long long* bad, unsigned long long* nan_bad) {
  return guard([&] { *bad = k::bf16_check_encode(nan_bad); });
}

int uh_mx_check_dequant(unsigned long long* bad, unsigned long long* total) {
  return guard([&] { *bad = k::mx_check_dequant(total); });
}

int uh_mx_grouped_gemv(const uint16_t* xa, int K, const int32_t* tiles, int ntiles, const uint8_t* const* w_tab,
                       const uint8_t* const* s_tab, uint16_t* out, int ldo, int N, void* st, const int* ntiles_dev,
                       const uint8_t* const* w_tab2, const uint8_t* const* s_tab2, uint16_t* out2, int max_rows,
                       const float* glu_w, const int32_t* glu_row_expert, const uint8_t* const* glu_s_tab,
                       uint16_t* glu_hh, float glu_limit, uint32_t* glu_counters) {
  return guard([&] {
    k::MxGlu glu{glu_w, glu_row_expert, glu_s_tab, glu_hh, glu_limit, glu_counters};
    k::mx_grouped_gemv(xa, K, T3(tiles), ntiles, w_tab, s_tab, out, ldo, N, S(st), ntiles_dev, w_tab2, s_tab2, out2,
                       max_rows, glu);
  });
}
int uh_mx_grouped_gemv_sums(const uint16_t* xa, int K, const int32_t* tiles, int ntiles, const uint8_t* const* w_tab,
                            const uint8_t* const* s_tab, uint16_t* out, int ldo, int N, void* st,
                            const int* ntiles_dev, int max_rows, const int32_t* sums_u2p, const int32_t* sums_plan,
                            int sums_K, uint16_t* sums_dst, uint32_t* sums_counters) {
  return guard([&] {
    k::MxSums sums{sums_u2p, reinterpret_cast<const k::MoePlan*>(sums_plan), sums_K, sums_dst, sums_counters};
    k::mx_grouped_gemv(xa, K, T3(tiles), ntiles, w_tab, s_tab, out, ldo, N, S(st), ntiles_dev, nullptr, nullptr,
                       nullptr, max_rows, k::MxGlu{}, sums);
  });
}
int uh_mx_grouped_gemm(const uint16_t* xa, int K, const int32_t* tiles, int ntiles, const uint8_t* const* w_tab,
                       const uint8_t* const* s_tab, uint16_t* out, int ldo, int N, void* st, const int* ntiles_dev,
                       const uint8_t* const* w_tab2, const uint8_t* const* s_tab2, uint16_t* out2, int max_rows) {
  return guard([&] {
    k::mx_grouped_gemm(xa, K, T3(tiles), ntiles, w_tab, s_tab, out, ldo, N, S(st), ntiles_dev, w_tab2, s_tab2, out2,
                       max_rows);
  });
}
int uh_mx_grouped_gemm_glu(const uint16_t* xa, int K, const int32_t* tiles, int ntiles, const uint8_t* const* w1_tab,
                           const uint8_t* const* s1_tab, const uint8_t* const* w3_tab, const uint8_t* const* s3_tab,
                           int N, const float* glu_w, const int32_t* glu_row_expert, const uint8_t* const* glu_s_tab,
                           uint16_t* glu_hh, float glu_limit, void* st, const int* ntiles_dev) {
  return guard([&] {
    k::MxGlu glu{glu_w, glu_row_expert, glu_s_tab, glu_hh, glu_limit, nullptr};
    k::mx_grouped_gemm_glu(xa, K, T3(tiles), ntiles, w1_tab, s1_tab, w3_tab, s3_tab, N, glu, S(st), ntiles_dev);
  });
}
int uh_mx_grouped_gemv_q(const uint8_t* q, const uint8_t* qs, int K, const int32_t* tiles, int ntiles,
                         const uint8_t* const* w_tab, const uint8_t* const* s_tab, uint16_t* out, int ldo, int N,
                         void* st, const int* ntiles_dev, const uint8_t* const* w_tab2, const uint8_t* const* s_tab2,
                         uint16_t* out2, int max_rows, const float* glu_w, const int32_t* glu_row_expert,
                         const uint8_t* const* glu_s_tab, uint16_t* glu_hh, uint8_t* glu_hq, uint8_t* glu_hs,
                         float glu_limit) {
  return guard([&] {
    k::MxGlu glu{glu_w, glu_row_expert, glu_s_tab, glu_hh, glu_limit, nullptr, glu_hq, glu_hs};
    k::mx_grouped_gemv_q(q, qs, K, T3(tiles), ntiles, w_tab, s_tab, out, ldo, N, S(st), ntiles_dev, w_tab2, s_tab2,
                         out2, max_rows, glu);
  });
}
int uh_mx_grouped_gemv_x(const uint16_t* x, int ldx, const int32_t* x_rows, int K, const int32_t* tiles, int ntiles,
                         const uint8_t* const* w_tab, const uint8_t* const* s_tab, uint16_t* out, int ldo, int N,
                         void* st, const int* ntiles_dev, const uint8_t* const* w_tab2, const uint8_t* const* s_tab2,
                         uint16_t* out2, int max_rows, const float* glu_w, const int32_t* glu_row_expert,
                         const uint8_t* const* glu_s_tab, uint16_t* glu_hh, uint8_t* glu_hq, uint8_t* glu_hs,
                         float glu_limit) {
  return guard([&] {
    k::MxGlu glu{glu_w, glu_row_expert, glu_s_tab, glu_hh, glu_limit, nullptr, glu_hq, glu_hs};
    k::mx_grouped_gemv_x(x, ldx, x_rows, K, T3(tiles), ntiles, w_tab, s_tab, out, ldo, N, S(st), ntiles_dev, w_tab2,
                         s_tab2, out2, max_rows, glu);
  });
}
int uh_mx_grouped_gemm_x(const uint16_t* x, int ldx, const int32_t* x_rows, int K, const int32_t* tiles, int ntiles,
                         const uint8_t* const* w_tab, const uint8_t* const* s_tab, uint16_t* out, int ldo, int N,
                         void* st, const int* ntiles_dev, const uint8_t* const* w_tab2, const uint8_t* const* s_tab2,
                         uint16_t* out2, const float* glu_w, const int32_t* glu_row_expert,
                         const uint8_t* const* glu_s_tab, uint16_t* glu_hh, uint8_t* glu_hq, uint8_t* glu_hs,
                         float glu_limit) {
  return guard([&] {
    k::MxGlu glu{glu_w, glu_row_expert, glu_s_tab, glu_hh, glu_limit, nullptr, glu_hq, glu_hs};
    k::mx_grouped_gemm_x(x, ldx, x_rows, K, T3(tiles), ntiles, w_tab, s_tab, out, ldo, N, S(st), ntiles_dev, w_tab2,
                         s_tab2, out2, glu);
  });
}
int uh_mx_grouped_gemm_q_f32out(const uint8_t* q, const uint8_t* qs, int K, const int32_t* tiles, int ntiles,
                                const uint8_t* const* w_tab, const uint8_t* const* s_tab, float* out, int ldo, int N,
                                void* st, const int* ntiles_dev) {
  return guard([&] {
    k::mx_grouped_gemm_q_f32out(q, qs, K, T3(tiles), ntiles, w_tab, s_tab, out, ldo, N, S(st), ntiles_dev);
  });
}
int uh_mx_gemm_set_exact(int on) { return k::mx_gemm_set_exact(on); }
int uh_mx_grouped_gemv_q_f32out(const uint8_t* q, const uint8_t* qs, int K, const int32_t* tiles, int ntiles,
                                const uint8_t* const* w_tab, const uint8_t* const* s_tab, float* out, int ldo, int N,
                                void* st, const int* ntiles_dev, int max_rows) {
  return guard([&] {
    k::mx_grouped_gemv_q_f32out(q, qs, K, T3(tiles), ntiles, w_tab, s_tab, out, ldo, N, S(st), ntiles_dev, max_rows);
  });
}
int uh_mx_grouped_gemm_q(const uint8_t* q, const uint8_t* qs, int K, const int32_t* tiles, int ntiles,
                         const uint8_t* const* w_tab, const uint8_t* const* s_tab, uint16_t* out, int ldo, int N,
                         void* st, const int* ntiles_dev, const uint8_t* const* w_tab2, const uint8_t* const* s_tab2,
                         uint16_t* out2, int max_rows, const float* glu_w, const int32_t* glu_row_expert,
                         const uint8_t* const* glu_s_tab, uint16_t* glu_hh, uint8_t* glu_hq, uint8_t* glu_hs,
                         float glu_limit) {
  return guard([&] {
    k::MxGlu glu{glu_w, glu_row_expert, glu_s_tab, glu_hh, glu_limit, nullptr, glu_hq, glu_hs};
    k::mx_grouped_gemm_q(q, qs, K, T3(tiles), ntiles, w_tab, s_tab, out, ldo, N, S(st), ntiles_dev, w_tab2, s_tab2,
                         out2, max_rows, glu);
  });
}

int uh_route(const float* logits, const float* bias, const int32_t* tid2eid, const int32_t* ids, int32_t* sel,
             float* weights, int T, int E, int K, float route_scale, void* st, const float* bias_vl, int vocab) {
  return guard([&] { k::route(logits, bias, tid2eid, ids, sel, weights, T, E, K, route_scale, S(st), bias_vl, vocab); });
}
int uh_route_fast(const float* logits, const float* bias, const int32_t* tid2eid, const int32_t* ids, int32_t* sel,
                  float* weights, int T, int E, int K, float route_scale, void* st, const float* bias_vl, int vocab) {
  return guard(
      [&] { k::route_fast(logits, bias, tid2eid, ids, sel, weights, T, E, K, route_scale, S(st), bias_vl, vocab); });
}
int uh_route_glm(const float* logits, const float* bias, int32_t* sel, float* weights, int T, int E, int K,
                 float route_scale, void* st) {
  return guard([&] { k::route_glm(logits, bias, sel, weights, T, E, K, route_scale, S(st)); });
}
int uh_route_softmax(const float* logits, int32_t* sel, float* weights, int T, int E, int K, void* st) {
  return guard([&] { k::route_softmax(logits, sel, weights, T, E, K, S(st)); });
}
int uh_moe_count(const int32_t* sel, int T, int K, int32_t* count, int E, void* st, uint32_t* hist) {
  return guard([&] { k::moe_count(sel, T, K, count, E, S(st), hist); });
}
int uh_moe_plan(int32_t* count, const uint8_t* resident, int E, int P, int32_t* plan, int32_t* local_tiles,
                int32_t* remote_tiles, int32_t* off, int32_t* fill, int max_tiles, void* st, int tile_rows) {
  return guard([&] {
    k::moe_plan(count, resident, E, P, reinterpret_cast<k::MoePlan*>(plan), reinterpret_cast<k::Exl3Tile*>(local_tiles),
                reinterpret_cast<k::Exl3Tile*>(remote_tiles), off, fill, max_tiles, S(st), tile_rows);
  });
}
int uh_moe_scatter(const int32_t* sel, const float* wt, int T, int K, const int32_t* off, int32_t* fill,
                   int32_t* eidx, float* ewt, int32_t* row_expert, int32_t* pidx, void* st) {
  return guard([&] { k::moe_scatter(sel, wt, T, K, off, fill, eidx, ewt, row_expert, pidx, S(st)); });
}
namespace {
k::MoeSmallArgs small_args(const int32_t* sel, const float* wt, int T, int K, int E, int P, int max_tiles,
                           int tile_rows, int32_t* plan, int32_t* tiles, int32_t* eidx, float* ewt,
                           int32_t* row_expert, int32_t* pidx, uint32_t* hist, const float* route_logits,
                           const float* route_bias, float route_scale, const float* ds_logits, const float* ds_bias,
                           const float* ds_bias_vl, const int32_t* ds_tid2eid, const int32_t* ids, int vocab) {
  k::MoeSmallArgs a{};
  a.sel = sel;
  a.wt = wt;
  a.T = T;
  a.K = K;
  a.hist = hist;
  a.E = E;
  a.P = P;
  a.max_tiles = max_tiles;
  a.tile_rows = tile_rows;
  a.plan = reinterpret_cast<k::MoePlan*>(plan);
  a.lt = reinterpret_cast<k::Exl3Tile*>(tiles);
  a.eidx = eidx;
  a.ewt = ewt;
  a.row_expert = row_expert;
  a.pidx = pidx;
  a.route_logits = route_logits;
  a.route_bias = route_bias;
  a.route_scale = route_scale;
  a.ds_logits = ds_logits;
  a.ds_bias = ds_bias;
  a.ds_bias_vl = ds_bias_vl;
  a.ds_tid2eid = ds_tid2eid;
  a.ids = ids;
  a.vocab = vocab;
  return a;
}
}  // namespace
int uh_moe_dispatch_small(const int32_t* sel, const float* wt, int T, int K, int E, int P, int max_tiles,
                          int tile_rows, int32_t* plan, int32_t* tiles, int32_t* eidx, float* ewt,
                          int32_t* row_expert, int32_t* pidx, uint32_t* hist, const float* route_logits,
                          const float* route_bias, float route_scale, const float* ds_logits, const float* ds_bias,
                          const float* ds_bias_vl, const int32_t* ds_tid2eid, const int32_t* ids, int vocab,
                          void* st) {
  return guard([&] {
    k::moe_dispatch_small(small_args(sel, wt, T, K, E, P, max_tiles, tile_rows, plan, tiles, eidx, ewt, row_expert,
                                     pidx, hist, route_logits, route_bias, route_scale, ds_logits, ds_bias, ds_bias_vl,
                                     ds_tid2eid, ids, vocab),
                          S(st));
  });
}
int uh_moe_dispatch_mid(const int32_t* sel, const float* wt, int T, int K, int E, int P, int max_tiles, int tile_rows,
                        int32_t* plan, int32_t* tiles, int32_t* eidx, float* ewt, int32_t* row_expert, int32_t* pidx,
                        uint32_t* hist, const float* route_logits, const float* route_bias, float route_scale,
                        const float* ds_logits, const float* ds_bias, const float* ds_bias_vl,
                        const int32_t* ds_tid2eid, const int32_t* ids, int vocab, const float* softmax_logits,
                        void* st) {
  return guard([&] {
    k::MoeSmallArgs a = small_args(sel, wt, T, K, E, P, max_tiles, tile_rows, plan, tiles, eidx, ewt, row_expert,
                                   pidx, hist, route_logits, route_bias, route_scale, ds_logits, ds_bias, ds_bias_vl,
                                   ds_tid2eid, ids, vocab);
    a.softmax_logits = softmax_logits;
    k::moe_dispatch_mid(a, S(st));
  });
}
int uh_swiglu(const uint16_t* gate, const uint16_t* up, const float* w, uint16_t* h, int rows, int dim, float limit,
              void* st) {
  return guard([&] { k::swiglu(gate, up, w, h, rows, dim, limit, S(st)); });
}
int uh_scatter_add(const uint16_t* src, const int32_t* rows_idx, float* y, int n, int dim, void* st) {
  return guard([&] { k::scatter_add(src, rows_idx, y, n, dim, S(st)); });
}
int uh_gather_rows(const uint16_t* src, const int32_t* rows_idx, uint16_t* dst, int n, int dim, void* st) {
  return guard([&] { k::gather_rows(src, rows_idx, dst, n, dim, S(st)); });
}
int uh_moe_combine(const uint16_t* pair_out, const int32_t* pidx, const uint16_t* shared, uint16_t* out, int T, int K,
                   int dim, void* st) {
  return guard([&] { k::moe_combine(pair_out, pidx, shared, out, T, K, dim, S(st)); });
}

int uh_act_quant_fp8(const uint16_t* x, int ldx, uint8_t* q, uint8_t* s, int rows, int cols, int block, void* st) {
  return guard([&] { k::act_quant_fp8(x, ldx, q, s, rows, cols, block, S(st)); });
}
int uh_fake_quant_fp8(uint16_t* x, int ldx, int rows, int cols, int block, void* st) {
  return guard([&] { k::fake_quant_fp8(x, ldx, rows, cols, block, S(st)); });
}
int uh_fake_quant_fp4(uint16_t* x, int ldx, int rows, int cols, int block, void* st) {
  return guard([&] { k::fake_quant_fp4(x, ldx, rows, cols, block, S(st)); });
}
int uh_act_quant_fp8_f32s(const uint16_t* x, int ldx, uint8_t* q, float* s, int rows, int cols, int block, void* st) {
  return guard([&] { k::act_quant_fp8_f32s(x, ldx, q, s, rows, cols, block, S(st)); });
}
int uh_gemm_w8a8(const uint8_t* a, const uint8_t* sa, const uint8_t* w, const uint8_t* sw, uint16_t* c, int ldc,
                 int M, int N, int K, void* st) {
  return guard([&] { k::gemm_w8a8(a, sa, w, sw, c, ldc, M, N, K, S(st)); });
}
int uh_gemm_w8a8_wmma(const uint8_t* a, const uint8_t* sa, const uint8_t* w, const uint8_t* sw, uint16_t* c, int ldc,
                      int M, int N, int K, void* st) {
  return guard([&] { k::gemm_w8a8_wmma(a, sa, w, sw, c, ldc, M, N, K, S(st)); });
}
int uh_gemv_w8a8(const uint8_t* a, const uint8_t* sa, const uint8_t* w, const uint8_t* sw, uint16_t* c, int ldc,
                 int M, int N, int K, void* st) {
  return guard([&] { k::gemv_w8a8(a, sa, w, sw, c, ldc, M, N, K, S(st)); });
}
int uh_gemv_w8a8_parts(const uint8_t* a, const uint8_t* sa, const void* const* w, const uint8_t* const* sw,
                       void* const* c, const int* ldc, const int* N, int nparts, int M, int K, void* st) {
  return guard([&] {
    if (!w || !sw || !c || !ldc || !N || nparts < 1 || nparts > k::GemvParts::kMax)
      throw std::runtime_error("uh_gemv_w8a8_parts: 1..3 parts");
    k::GemvPart parts[k::GemvParts::kMax];
    for (int i = 0; i < nparts; ++i) parts[i] = k::GemvPart{w[i], sw[i], c[i], ldc[i], N[i]};
    k::gemv_w8a8_parts(a, sa, parts, nparts, M, K, S(st));
  });
}
int uh_gemv_w8a8_glu(const uint8_t* a, const uint8_t* sa, const uint8_t* w_gate, const uint8_t* sw_gate,
                     uint16_t* gate, int ldg, const uint8_t* w_up, const uint8_t* sw_up, uint16_t* up, int ldu, int I,
                     int M, int K, float limit, uint8_t* q, uint8_t* qs, uint32_t* counters, void* st) {
  return guard([&] {
    const k::GemvPart parts[2] = {{w_gate, sw_gate, gate, ldg, I}, {w_up, sw_up, up, ldu, I}};
    k::gemv_w8a8_glu(a, sa, parts, M, K, limit, k::GemvQuant{q, qs, counters}, S(st));
  });
}
int uh_gemm_fp8_f32s(const uint8_t* a, const float* sa, const uint8_t* w, const float* sw, uint16_t* c, int ldc,
                     int M, int N, int K, void* st) {
  return guard([&] { k::gemm_fp8_f32s(a, sa, w, sw, c, ldc, M, N, K, S(st)); });
}
uint64_t uh_pack_xxh64(const void* data, size_t len, uint64_t seed) { return unholy::model::pack::xxh64(data, len, seed); }
int uh_pack_write(const char* path, int n_layers, int n_mtp, int n_experts, int w13_out, int w13_in, int w2_out,
                  int w2_in, const uint8_t* const* parts, uint64_t config_hash, uint64_t source_hash) {
  namespace pk = unholy::model::pack;
  return guard([&] {
    pk::write_pack(path, pk::geometry_for(n_layers, n_mtp, n_experts, w13_out, w13_in, w2_out, w2_in), parts,
                   config_hash, source_hash);
  });
}
int uh_pack_read_header(const char* path, uint8_t* header) {
  namespace pk = unholy::model::pack;
  return guard([&] {
    const int fd = ::open(path, O_RDONLY);
    if (fd < 0) throw std::runtime_error(std::string("expert pack: cannot open ") + path);
    try {
      const pk::Header h = pk::read_header(fd);
      std::memcpy(header, &h, sizeof h);
    } catch (...) {
      ::close(fd);
      throw;
    }
    ::close(fd);
  });
}
int uh_pack_load(const char* path, size_t first, size_t count, void* dst, size_t stride, int verify, int direct,
                 void* st) {
  namespace pk = unholy::model::pack;
  return guard([&] {
    const int fd = ::open(path, O_RDONLY | (direct ? O_DIRECT : 0));
    if (fd < 0) throw std::runtime_error(std::string("expert pack: cannot open ") + path);
    try {
      pk::load_slots(fd, pk::read_header(fd), first, count, dst, stride, verify != 0, st);
    } catch (...) {
      ::close(fd);
      throw;
    }
    ::close(fd);
  });
}
int uh_pack_expert_table(const uint8_t* header, const void* slots, size_t stride, int E, uint64_t* tab) {
  namespace pk = unholy::model::pack;
  return guard([&] {
    pk::Header h;
    std::memcpy(&h, header, sizeof h);
    if (!slots || !tab || E <= 0 || stride < h.slot_bytes) throw std::runtime_error("expert pack: table arguments");
    for (int e = 0; e < E; ++e)
      for (int f = 0; f < pk::kParts; ++f)
        tab[size_t(f) * E + e] = uint64_t(reinterpret_cast<uintptr_t>(slots) + e * stride + h.part_offset[f]);
  });
}
int uh_rmsnorm_quant_slices(const uint16_t* x, int ldx, const uint16_t* w, uint16_t* y, int ldy, uint8_t* q,
                            uint8_t* qs, int rows, int dim, float eps, int* launched, void* st) {
  return guard([&] {
    const bool done = k::rmsnorm_quant_slices(x, ldx, w, y, ldy, q, qs, rows, dim, eps, S(st));
    if (launched) *launched = done ? 1 : 0;
  });
}
int uh_quant_remote_tokens(const uint16_t* x, int dim, const int32_t* u2t, const int32_t* plan, uint8_t* q, uint8_t* s,
                           int max_tokens, void* st) {
  return guard([&] {
    k::quant_remote_tokens(x, dim, u2t, reinterpret_cast<const k::MoePlan*>(plan), q, s, max_tokens, S(st));
  });
}
int uh_mx_xform_in_q(const uint8_t* q, const uint8_t* s, const int32_t* p2u, const int32_t* plan,
                     const int32_t* row_expert, const uint8_t* const* s_tab, uint16_t* xa, int P, int K, void* st) {
  return guard([&] {
    k::mx_xform_in_q(q, s, p2u, reinterpret_cast<const k::MoePlan*>(plan), row_expert, s_tab, xa, P, K, S(st));
  });
}
int uh_mx_xform_in_q_fp8(const uint8_t* q, const uint8_t* s, const int32_t* p2u, const int32_t* plan,
                         const int32_t* row_expert, const uint8_t* const* s_tab, uint8_t* qo, uint8_t* qso, int P,
                         int K, void* st) {
  return guard([&] {
    k::mx_xform_in_q_fp8(q, s, p2u, reinterpret_cast<const k::MoePlan*>(plan), row_expert, s_tab, qo, qso, P, K,
                         S(st));
  });
}
int uh_moe_trace(const int32_t* sel, int n, uint8_t* dst, void* st) {
  return guard([&] { k::moe_trace(sel, n, dst, S(st)); });
}
int uh_rmsnorm_slices(const uint16_t* x, int ldx, const uint16_t* w, uint16_t* y, int ldy, int rows, int dim, float eps,
                      void* st) {
  return guard([&] { k::rmsnorm_slices(x, ldx, w, y, ldy, rows, dim, eps, S(st)); });
}
int uh_hc_post_slices(const uint16_t* x, const uint16_t* res, const float* post, const float* comb, uint16_t* out,
                      int T, int hc, int dim, void* st) {
  return guard([&] { k::hc_post_slices(x, res, post, comb, out, T, hc, dim, S(st)); });
}
int uh_copy_remote_rows(const uint16_t* src, uint16_t* dst, const int32_t* plan, int dim, int max_rows, void* st) {
  return guard([&] { k::copy_remote_rows(src, dst, reinterpret_cast<const k::MoePlan*>(plan), dim, max_rows, S(st)); });
}
int uh_stage_remote(const int32_t* plan, const int32_t* rtiles, const float* ewt, const int32_t* row_expert,
                    int32_t* plan_dst, int32_t* tiles_dst, float* w_dst, int32_t* e_dst, int max_rows, void* st) {
  return guard([&] {
    k::stage_remote(reinterpret_cast<const k::MoePlan*>(plan), reinterpret_cast<const k::Exl3Tile*>(rtiles), ewt,
                    row_expert, reinterpret_cast<k::MoePlan*>(plan_dst), reinterpret_cast<k::Exl3Tile*>(tiles_dst),
                    w_dst, e_dst, max_rows, S(st));
  });
}
int uh_copy_remote_meta(const float* ewt, const int32_t* row_expert, float* w_dst, int32_t* e_dst, const int32_t* plan,
                        int max_rows, void* st) {
  return guard([&] {
    k::copy_remote_meta(ewt, row_expert, w_dst, e_dst, reinterpret_cast<const k::MoePlan*>(plan), max_rows, S(st));
  });
}
int uh_remote_tokens(const int32_t* pidx, const int32_t* eidx, int T, int K, int32_t* plan, int32_t* tok2u,
                     int32_t* u2t, int32_t* p2u, int32_t* u2p, void* st) {
  return guard([&] {
    k::remote_tokens(pidx, eidx, T, K, reinterpret_cast<k::MoePlan*>(plan), tok2u, u2t, p2u, u2p, S(st));
  });
}
int uh_remote_combine(const uint16_t* pair_out, const int32_t* u2p, const int32_t* plan, uint16_t* dst, int K, int dim,
                      int max_tokens, void* st) {
  return guard([&] {
    k::remote_combine(pair_out, u2p, reinterpret_cast<const k::MoePlan*>(plan), dst, K, dim, max_tokens, S(st));
  });
}
int uh_copy_remote_tokens(const uint16_t* x, int dim, const int32_t* u2t, const int32_t* plan, uint16_t* dst,
                          int max_tokens, void* st) {
  return guard([&] {
    k::copy_remote_tokens(x, dim, u2t, reinterpret_cast<const k::MoePlan*>(plan), dst, max_tokens, S(st));
  });
}
int uh_copy_remote_partial(const uint16_t* src, uint16_t* dst, const int32_t* plan, int dim, int max_tokens,
                           void* st) {
  return guard([&] {
    k::copy_remote_partial(src, dst, reinterpret_cast<const k::MoePlan*>(plan), dim, max_tokens, S(st));
  });
}
int uh_moe_combine_partial(const uint16_t* pair_out, const int32_t* pidx, const int32_t* plan, const int32_t* tok2u,
                           const uint16_t* shared, uint16_t* out, int T, int K, int dim, void* st) {
  return guard([&] {
    k::moe_combine_partial(pair_out, pidx, reinterpret_cast<const k::MoePlan*>(plan), tok2u, shared, out, T, K, dim,
                           S(st));
  });
}
int uh_moe_combine_partial_link(const uint16_t* pair_out, const int32_t* pidx, const int32_t* plan,
                                const int32_t* tok2u, const uint16_t* remote, const uint16_t* shared, uint16_t* out,
                                int T, int K, int dim, uint16_t* hc_x, const float* post, const float* comb, int hc,
                                void* st) {
  return guard([&] {
    k::HcPostArgs hp;
    hp.x = hc_x;
    hp.post = post;
    hp.comb = comb;
    hp.hc = hc;
    k::moe_combine_partial_link(pair_out, pidx, reinterpret_cast<const k::MoePlan*>(plan), tok2u, remote, shared, out,
                                T, K, dim, S(st), hp);
  });
}
int uh_moe_dispatch_small_remote(const int32_t* sel, const float* wt, int T, int K, int E, int P, int max_tiles,
                                 int tile_rows, int32_t* plan, int32_t* tiles, int32_t* remote_tiles, int32_t* eidx,
                                 float* ewt, int32_t* row_expert, int32_t* pidx, const uint8_t* resident,
                                 const float* ds_logits, const float* ds_bias, float route_scale, int remote, int qin,
                                 int32_t* tok2u, int32_t* u2t, int32_t* p2u, int32_t* u2p, int32_t* plan_dst,
                                 int32_t* tiles_dst, float* w_dst, int32_t* e_dst, const uint16_t* x, int dim,
                                 uint16_t* x_dst, uint8_t* q_dst, uint8_t* qs_dst, uint32_t* req_flag,
                                 uint32_t req_value, void* st) {
  return guard([&] {
    k::MoeSmallArgs a{};
    a.sel = sel;
    a.wt = wt;
    a.T = T;
    a.K = K;
    a.resident = resident;
    a.E = E;
    a.P = P;
    a.max_tiles = max_tiles;
    a.tile_rows = tile_rows;
    a.plan = reinterpret_cast<k::MoePlan*>(plan);
    a.lt = reinterpret_cast<k::Exl3Tile*>(tiles);
    a.rtl = reinterpret_cast<k::Exl3Tile*>(remote_tiles);
    a.eidx = eidx;
    a.ewt = ewt;
    a.row_expert = row_expert;
    a.pidx = pidx;
    a.ds_logits = ds_logits;
    a.ds_bias = ds_bias;
    a.route_scale = route_scale;
    a.remote = remote != 0;
    a.qin = qin != 0;
    a.tok2u = tok2u;
    a.u2t = u2t;
    a.p2u_dst = p2u;
    a.u2p_dst = u2p;
    a.plan_dst = reinterpret_cast<k::MoePlan*>(plan_dst);
    a.tiles_dst = reinterpret_cast<k::Exl3Tile*>(tiles_dst);
    a.w_dst = w_dst;
    a.e_dst = e_dst;
    a.x = x;
    a.dim = dim;
    a.x_dst = x_dst;
    a.q_dst = q_dst;
    a.qs_dst = qs_dst;
    a.req_flag = req_flag;
    a.req_value = req_value;
    k::moe_dispatch_small(a, S(st));
  });
}
int uh_gemm_grouped_fp8w(const uint16_t* a, const uint8_t* w, const uint8_t* sw, uint16_t* c, int M, int G, int R,
                         int K, void* st) {
  return guard([&] { k::gemm_grouped_fp8w(a, w, sw, c, M, G, R, K, S(st)); });
}
int uh_gemm_grouped_fp8w_wmma(const uint16_t* a, const uint8_t* w, const uint8_t* sw, uint16_t* c, int M, int G,
                              int R, int K, void* st) {
  return guard([&] { k::gemm_grouped_fp8w_wmma(a, w, sw, c, M, G, R, K, S(st)); });
}
int uh_gemv_grouped_fp8w(const uint16_t* a, const uint8_t* w, const uint8_t* sw, uint16_t* c, int M, int G, int R,
                         int K, uint8_t* q, uint8_t* qs, uint32_t* counters, void* st) {
  return guard([&] { k::gemv_grouped_fp8w(a, w, sw, c, M, G, R, K, S(st), k::GemvQuant{q, qs, counters}); });
}
int uh_gemm_fp8_f32s_x(const uint16_t* x, int ldx, const uint8_t* w, const float* sw, uint16_t* c, int ldc, int M,
                       int N, int K, void* st) {
  return guard([&] { k::gemm_fp8_f32s_x(x, ldx, w, sw, c, ldc, M, N, K, S(st)); });
}
int uh_gemm_a8w4(const uint8_t* a, const uint8_t* sa, const uint8_t* w, const uint8_t* sw, uint16_t* c, int ldc,
                 int M, int N, int K, void* st) {
  return guard([&] { k::gemm_a8w4(a, sa, w, sw, c, ldc, M, N, K, S(st)); });
}
int uh_gemm_a8w4_tiled(const uint8_t* a, const uint8_t* sa, const uint8_t* w, const uint8_t* sw, uint16_t* c, int ldc,
                       int M, int N, int K, void* st) {
  return guard([&] { k::gemm_a8w4_tiled(a, sa, w, sw, c, ldc, M, N, K, S(st)); });
}
int uh_quant_weight_fp8_f32s(const float* w, uint8_t* q, float* s, int N, int K, void* st) {
  return guard([&] {
    if (K % 128 || N <= 0) throw std::runtime_error("uh_quant_weight_fp8_f32s: K % 128");
    quant_weight_kernel<<<dim3(unsigned(K / 128), uh::cdiv(size_t(N), 128)), 256, 0, S(st)>>>(w, q, s, N, K);
    UH_CHECK_LAUNCH();
  });
}

int uh_exp_f32_array(const float* x, float* y, size_t n, void* st) {
  return guard([&] {
    if (!n) return;
    exp_f32_kernel<<<std::min<unsigned>(uh::cdiv(n, 256), 4096u), 256, 0, S(st)>>>(x, y, n);
    UH_CHECK_LAUNCH();
  });
}

size_t uh_mx_moe_workspace_size(int T, int K, int E, int D, int I) { return carve(nullptr, T, K, E, D, I).bytes; }

int uh_mx_moe_forward(const uint16_t* x, const float* logits, int T, int K, int E, int D, int I,
                      const uint8_t* const* tab, float limit, void* ws, size_t ws_bytes, uint16_t* out, int32_t* sel,
                      float* wt, void* stream) {
  return uh_mx_moe_forward_ev(x, logits, T, K, E, D, I, tab, limit, ws, ws_bytes, out, sel, wt, stream, nullptr);
}

int uh_mx_moe_forward_ev(const uint16_t* x, const float* logits, int T, int K, int E, int D, int I,
                         const uint8_t* const* tab, float limit, void* ws, size_t ws_bytes, uint16_t* out, int32_t* sel,
                         float* wt, void* stream, void* const* events) {
  return guard([&] {
    const auto mark = [&](int i) {
      if (events && events[i]) UH_CHECK(hipEventRecord(static_cast<hipEvent_t>(events[i]), static_cast<hipStream_t>(stream)));
    };
    if (T <= 0) return;
    const MoeWs w = carve(static_cast<char*>(ws), T, K, E, D, I);
    if (ws_bytes < w.bytes) throw std::runtime_error("uh_mx_moe_forward: workspace too small");
    if (D % 128 || I % 128) throw std::runtime_error("uh_mx_moe_forward: D % 128, I % 128");
    const hipStream_t st = S(stream);
    const int P = T * K;
    int32_t* s_sel = sel ? sel : w.sel;
    float* s_wt = wt ? wt : w.wt;
    const auto t = [&](int m, int f) { return tab + size_t(2 * m + f) * E; };
    mark(0);
    // Dispatch in one single-block launch up to 512 picks; the routing in that launch too while every token has a
    // wave of its own (T <= 8), else a wave per token over many workgroups first.
    const bool one_block = P <= k::kMoeMidMaxPicks, route_in = one_block && T <= 8;
    if (!route_in) k::route_softmax(logits, s_sel, s_wt, T, E, K, st);
    const int* ntd = &reinterpret_cast<const k::MoePlan*>(w.plan)->n_local_tiles;
    k::Exl3Tile* tiles = reinterpret_cast<k::Exl3Tile*>(w.tiles);
    if (one_block) {
      k::MoeSmallArgs a{};
      a.sel = s_sel;
      a.wt = s_wt;
      a.T = T;
      a.K = K;
      a.E = E;
      a.P = P;
      a.max_tiles = w.max_tiles;
      a.tile_rows = w.tile_rows;
      a.plan = reinterpret_cast<k::MoePlan*>(w.plan);
      a.lt = tiles;
      a.eidx = w.eidx;
      a.ewt = w.ewt;
      a.row_expert = w.row_expert;
      a.pidx = w.pidx;
      a.softmax_logits = route_in ? logits : nullptr;
      k::moe_dispatch_mid(a, st);
    } else {
      k::launch_zero_words(w.count, size_t(E), st);  // a kernel: no memset node if the caller captures a graph
      k::moe_count(s_sel, T, K, w.count, E, st);
      k::moe_plan(w.count, nullptr, E, P, reinterpret_cast<k::MoePlan*>(w.plan), tiles, nullptr, w.off, w.fill,
                  w.max_tiles, st, w.tile_rows);
      k::moe_scatter_e(s_sel, s_wt, T, K, E, w.off, w.eidx, w.ewt, w.row_expert, w.pidx, st);
    }
    mark(1);
    const k::MxGlu glu{w.ewt, w.row_expert, t(2, 1), nullptr, limit, nullptr, w.hq, w.hs};
    if (T <= 64) {
      // Both GEMVs quantize their inputs while staging them: x rows per 128 for w1 / w3, and for w2 the raw SwiGLU
      // rows h, whose act_quant codes are exactly those of the fake-quantized hh. A tile holds at most one row per
      // token, so min(tile_rows, T) rows bound the staging.
      k::MxGlu gh = glu;
      gh.hq = gh.hs = nullptr;
      gh.h = w.h;
      const int rows = std::min(w.tile_rows, T);
      mark(2);
      k::mx_grouped_gemv_x(x, D, w.eidx, D, tiles, w.max_tiles, t(0, 0), t(0, 1), nullptr, I, I, st, ntd, t(1, 0),
                           t(1, 1), nullptr, rows, gh);
      mark(3);
      k::mx_grouped_gemv_x(w.h, I, nullptr, I, tiles, w.max_tiles, t(2, 0), t(2, 1), w.pair_out, D, D, st, ntd,
                           nullptr, nullptr, nullptr, rows, k::MxGlu{});
    } else if (!prefill_fp8() && k::mx_gemm_exact()) {
      // Each token row fake-quantized once to bf16 (exact e4m3 x 2^k values; its K picks would otherwise be
      // quantized K times); the w1 / w3 GEMM gathers the pair rows through eidx and writes the fake-quantized
      // SwiGLU rows hh, the w2 GEMM's bf16 input.
      k::mx_xform_in(x, D, nullptr, nullptr, w.xa, T, D, st, nullptr);
      mark(2);
      k::MxGlu gb = glu;
      gb.hq = gb.hs = nullptr;
      gb.hh = w.hh;
      k::mx_grouped_gemm_rows(w.xa, w.eidx, D, tiles, w.max_tiles, t(0, 0), t(0, 1), nullptr, I, I, st, ntd, t(1, 0),
                              t(1, 1), nullptr, gb);
      mark(3);
      k::mx_grouped_gemm_rows(w.hh, nullptr, I, tiles, w.max_tiles, t(2, 0), t(2, 1), w.pair_out, D, D, st, ntd);
    } else {
      // Each token row quantized once (its K picks would otherwise be quantized K times); the GEMM's loads gather
      // the pair rows' codes through eidx.
      k::mx_xform_in_fp8(x, D, nullptr, nullptr, w.xq, w.xs, T, D, st, nullptr);
      mark(2);
      k::mx_grouped_gemm_q(w.xq, w.xs, D, tiles, w.max_tiles, t(0, 0), t(0, 1), nullptr, I, I, st, ntd, t(1, 0), t(1, 1),
                           nullptr, w.tile_rows, glu, w.eidx);
      mark(3);
      k::mx_grouped_gemm_q(w.hq, w.hs, I, tiles, w.max_tiles, t(2, 0), t(2, 1), w.pair_out, D, D, st, ntd, nullptr,
                           nullptr, nullptr, w.tile_rows);
    }
    mark(4);
    k::moe_combine(w.pair_out, w.pidx, nullptr, out, T, K, D, st);
    mark(5);
  });
}

size_t uh_mx_moe_noalloc_max_bytes(void) { return kScratchBytes; }

int uh_mx_moe_forward_noalloc(const uint16_t* x, const float* logits, int T, int K, int E, int D, int I,
                              const uint8_t* const* tab, float limit, uint16_t* out, int32_t* sel, float* wt,
                              void* stream) {
  void* ws = nullptr;
  size_t need = 0;
  const int rc = guard([&] {
    need = carve(nullptr, T, K, E, D, I).bytes;
    if (need > kScratchBytes)
      throw std::runtime_error("uh_mx_moe_forward_noalloc: the workspace of T=" + std::to_string(T) + ", K=" +
                               std::to_string(K) + ", E=" + std::to_string(E) + ", D=" + std::to_string(D) +
                               ", I=" + std::to_string(I) + " is " + std::to_string(need) +
                               " bytes, above the fixed scratch of " + std::to_string(kScratchBytes) + " bytes");
    ws = scratch_ptr();
  });
  if (rc) return rc;
  return uh_mx_moe_forward_ev(x, logits, T, K, E, D, I, tab, limit, ws, kScratchBytes, out, sel, wt, stream, nullptr);
}

}  // extern "C"
