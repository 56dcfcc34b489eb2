// C entry points over the reference's own host code, compiled from its sources where they lie
// (/root/reference/src/core/half.hpp, /root/reference/src/model/expert_pack.cpp + safetensors.cpp, see the
// Makefile). TEST INFRASTRUCTURE ONLY: the tests use it to pin the oracle (uh_oracle.cpp) against the
// reference's host conversions and its CPU repack, and the expert pack (xxh64, header) against the reference's
// own; nothing in the product loads it.
#include <fcntl.h>
#include <unistd.h>

#include <cstdint>
#include <cstring>

#include "core/half.hpp"
#include "model/expert_pack.hpp"

extern "C" {
float ref_bf16_to_float(uint16_t b) { return unholy::bf16_to_float(b); }
float ref_e4m3_to_float(uint8_t v) { return unholy::e4m3_to_float(v); }
float ref_e8m0_to_float(uint8_t v) { return unholy::e8m0_to_float(v); }
float ref_e2m1_to_float(uint8_t v) { return unholy::e2m1_to_float(v); }
void ref_repack_matrix(const uint8_t* w, const uint8_t* s, uint8_t* tw, uint8_t* ts, int n, int k) {
  unholy::model::pack::repack_matrix(w, s, tw, ts, n, k);
}
void ref_unrepack_matrix(const uint8_t* tw, const uint8_t* ts, uint8_t* w, uint8_t* s, int n, int k) {
  unholy::model::pack::unrepack_matrix(tw, ts, w, s, n, k);
}
uint64_t ref_xxh64(const void* p, size_t n, uint64_t seed) { return unholy::model::pack::xxh64(p, n, seed); }
// The reference's read_header on a file: 0 and the header's bytes, or -1 where it throws.
int ref_read_header(const char* path, uint8_t* out) {
  const int fd = ::open(path, O_RDONLY);
  if (fd < 0) return -1;
  int rc = 0;
  try {
    const unholy::model::pack::Header h = unholy::model::pack::read_header(fd);
    std::memcpy(out, &h, sizeof h);
  } catch (...) {
    rc = -1;
  }
  ::close(fd);
  return rc;
}
int ref_header_size() { return int(sizeof(unholy::model::pack::Header)); }
}
