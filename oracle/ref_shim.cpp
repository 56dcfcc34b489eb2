// C entry points over the reference's own host code, compiled from its sources where they lie
// (/root/reference/src/core/half.hpp, /root/reference/src/model/expert_pack.cpp + safetensors.cpp, see the
// Makefile). TEST INFRASTRUCTURE ONLY: the tests use it to pin the oracle (uh_oracle.cpp) against the
// reference's host conversions and its CPU repack; nothing in the product loads it.
#include <cstdint>

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
}
