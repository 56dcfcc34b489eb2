// A C++ caller of the drop-in entry points, compiled against include/unholy/kernels/*.hpp and linked with
// libunholy_amd.so the way the reference's engine would be relinked: the reference's native-MXFP4 expert sequence
// (src/model/forward_ref.hip:455-470: mx_xform_in, the w1 / w3 launch with the SwiGLU epilogue writing hh, the w2
// launch on hh; routing and dispatch before it, moe_combine after) through the C++ API, checked bit for bit against
// the library's own forward (uh_mx_moe_forward, C ABI). Prints one line per case and exits nonzero on a mismatch.
//
//   build: tests/cpp/build.sh (hipcc, gfx950); run: tests/cpp/dropin_link (needs a GPU)
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "unholy/kernels/moe_dispatch.hpp"
#include "unholy/kernels/mx_moe.hpp"
#include "unholy/kernels/ref.hpp"
#include "unholy_amd.h"

namespace k = unholy::kernels;

#define CK(x)                                                                   \
  do {                                                                          \
    const hipError_t e_ = (x);                                                  \
    if (e_ != hipSuccess) {                                                     \
      std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));              \
      std::exit(2);                                                             \
    }                                                                           \
  } while (0)

namespace {

struct Lcg {  // splitmix64
  uint64_t s;
  uint64_t next() {
    uint64_t z = (s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
  }
  float normal() {  // sum of 4 uniforms, centred: a cheap bell shape is enough here
    float a = 0.0f;
    for (int i = 0; i < 4; ++i) a += float(next() >> 40) * (1.0f / 16777216.0f);
    return (a - 2.0f) * 1.7f;
  }
};

uint16_t to_bf16(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return uint16_t((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

template <class T>
T* dev(const std::vector<T>& h) {
  T* p = nullptr;
  CK(hipMalloc(&p, h.size() * sizeof(T)));
  CK(hipMemcpy(p, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
  return p;
}
template <class T>
T* dev_zero(size_t n) {
  T* p = nullptr;
  CK(hipMalloc(&p, n * sizeof(T)));
  CK(hipMemset(p, 0, n * sizeof(T)));
  return p;
}

// seq: 0 = the grouped GEMV with the SwiGLU epilogue (decode: tiles of 16 rows), 1 = the grouped GEMM with the
// SwiGLU epilogue (mx_grouped_gemm_glu, 128-row tiles), 2 = the gfx12 order of forward_ref.hip:459-470 for a verify
// step (UNHOLY_MX_GEMV_TOKENS unset, so T > 8 is not a GEMV step): w1 and w3 through mx_grouped_gemm with
// max_rows = T on 128-row tiles, mx_swiglu, then w2 through mx_grouped_gemm with max_rows = T.
int run_case(int T, int K, int E, int D, int I, uint64_t seed, int seq) {
  Lcg rng{seed};
  const float limit = 10.0f;
  const int P = T * K;
  // experts: w1, w3 [I, D], w2 [D, I] as row-major codes + scales, repacked on the device by mx_repack_to
  const int shapes[3][2] = {{I, D}, {I, D}, {D, I}};
  std::vector<const uint8_t*> tab(6 * size_t(E));
  for (int e = 0; e < E; ++e)
    for (int m = 0; m < 3; ++m) {
      const int N = shapes[m][0], Kd = shapes[m][1];
      std::vector<uint8_t> w(size_t(N) * Kd / 2), s(size_t(N) * Kd / 32);
      for (auto& b : w) b = uint8_t(rng.next());
      for (auto& b : s) b = uint8_t(119 + rng.next() % 7);
      uint8_t* dw = dev(w);
      uint8_t* ds = dev(s);
      uint8_t* tw = dev_zero<uint8_t>(w.size());
      uint8_t* ts = dev_zero<uint8_t>(s.size());
      k::mx_repack_to(dw, ds, tw, ts, N, Kd, nullptr);
      tab[size_t(2 * m) * E + e] = tw;
      tab[size_t(2 * m + 1) * E + e] = ts;
    }
  const uint8_t* const* dtab = dev(tab);
  const auto t = [&](int m, int f) { return dtab + size_t(2 * m + f) * E; };
  std::vector<uint16_t> x(size_t(T) * D);
  for (auto& v : x) v = to_bf16(rng.normal());
  std::vector<float> logits(size_t(T) * E);
  for (auto& v : logits) v = rng.normal();
  uint16_t* dx = dev(x);
  float* dl = dev(logits);

  // the reference's sequence through the C++ API
  int32_t* sel = dev_zero<int32_t>(P);
  float* wt = dev_zero<float>(P);
  k::route_softmax(dl, sel, wt, T, E, K, nullptr);
  const bool gemv = seq == 0;
  const int tile_rows = gemv ? 16 : k::kExl3TileRows, max_tiles = P + E;
  int32_t* count = dev_zero<int32_t>(E);
  int32_t* off = dev_zero<int32_t>(E);
  int32_t* fill = dev_zero<int32_t>(E);
  k::MoePlan* plan = dev_zero<k::MoePlan>(1);
  k::Exl3Tile* tiles = dev_zero<k::Exl3Tile>(max_tiles);
  int32_t* eidx = dev_zero<int32_t>(P);
  float* ewt = dev_zero<float>(P);
  int32_t* row_expert = dev_zero<int32_t>(P);
  int32_t* pidx = dev_zero<int32_t>(P);
  k::moe_count(sel, T, K, count, E, nullptr);
  k::moe_plan(count, nullptr, E, P, plan, tiles, nullptr, off, fill, max_tiles, nullptr, tile_rows);
  k::moe_scatter(sel, wt, T, K, off, fill, eidx, ewt, row_expert, pidx, nullptr);
  const int* ntd = &plan->n_local_tiles;
  uint16_t* xa = dev_zero<uint16_t>(size_t(P) * D);
  uint16_t* hh = dev_zero<uint16_t>(size_t(P) * I);
  uint16_t* gbuf = dev_zero<uint16_t>(size_t(P) * I);
  uint16_t* ubuf = dev_zero<uint16_t>(size_t(P) * I);
  uint16_t* pair = dev_zero<uint16_t>(size_t(P) * D);
  uint16_t* out = dev_zero<uint16_t>(size_t(T) * D);
  k::mx_xform_in(dx, D, row_expert, t(0, 1), xa, P, D, nullptr, eidx);
  const k::MxGlu glu{ewt, row_expert, t(2, 1), hh, limit, nullptr};
  const int rows = gemv ? std::min(T, tile_rows) : tile_rows;
  if (gemv) {
    k::mx_grouped_gemv(xa, D, tiles, max_tiles, t(0, 0), t(0, 1), nullptr, I, I, nullptr, ntd, t(1, 0), t(1, 1), nullptr,
                       rows, glu);
    k::mx_grouped_gemv(hh, I, tiles, max_tiles, t(2, 0), t(2, 1), pair, D, D, nullptr, ntd, nullptr, nullptr, nullptr,
                       rows);
  } else if (seq == 1) {
    k::mx_grouped_gemm_glu(xa, D, tiles, max_tiles, t(0, 0), t(0, 1), t(1, 0), t(1, 1), I, glu, nullptr, ntd);
    k::mx_grouped_gemm(hh, I, tiles, max_tiles, t(2, 0), t(2, 1), pair, D, D, nullptr, ntd);
  } else {
    const int vrows = std::min(T, k::kExl3TileRows);  // an expert has at most one row per token
    k::mx_grouped_gemm(xa, D, tiles, max_tiles, t(0, 0), t(0, 1), gbuf, I, I, nullptr, ntd, t(1, 0), t(1, 1), ubuf,
                       vrows);
    k::mx_swiglu(gbuf, ubuf, ewt, row_expert, t(2, 1), hh, P, I, limit, nullptr);
    k::mx_grouped_gemm(hh, I, tiles, max_tiles, t(2, 0), t(2, 1), pair, D, D, nullptr, ntd, nullptr, nullptr, nullptr,
                       vrows);
  }
  k::moe_combine(pair, pidx, nullptr, out, T, K, D, nullptr);

  // the library's forward through the C ABI
  const size_t ws_bytes = uh_mx_moe_workspace_size(T, K, E, D, I);
  void* ws = dev_zero<uint8_t>(ws_bytes);
  uint16_t* out2 = dev_zero<uint16_t>(size_t(T) * D);
  if (uh_mx_moe_forward(dx, dl, T, K, E, D, I, dtab, limit, ws, ws_bytes, out2, nullptr, nullptr, nullptr) != 0) {
    std::fprintf(stderr, "uh_mx_moe_forward: %s\n", uh_last_error());
    return 1;
  }
  CK(hipDeviceSynchronize());
  std::vector<uint16_t> a(size_t(T) * D), b(size_t(T) * D);
  CK(hipMemcpy(a.data(), out, a.size() * 2, hipMemcpyDeviceToHost));
  CK(hipMemcpy(b.data(), out2, b.size() * 2, hipMemcpyDeviceToHost));
  size_t diff = 0, nonzero = 0;
  for (size_t i = 0; i < a.size(); ++i) {
    diff += a[i] != b[i];
    nonzero += (a[i] & 0x7fff) != 0;
  }
  static const char* const names[3] = {"grouped GEMV", "grouped GEMM", "grouped GEMM, max_rows = T"};
  std::printf("dropin_link: T=%d K=%d E=%d D=%d I=%d (%s): %zu of %zu outputs differ, %zu nonzero\n", T, K, E, D, I,
              names[seq], diff, a.size(), nonzero);
  return diff == 0 && nonzero > a.size() / 2 ? 0 : 1;
}

}  // namespace

int main() {
  int bad = 0;
  bad |= run_case(8, 6, 32, 512, 256, 1, 0);
  bad |= run_case(200, 4, 16, 512, 256, 2, 1);
  bad |= run_case(64, 6, 32, 512, 256, 3, 2);
  std::printf("dropin_link: %s\n", bad ? "MISMATCH" : "OK");
  return bad;
}
