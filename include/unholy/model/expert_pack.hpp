// The expert pack: routed MXFP4 experts stored in the layout the grouped kernels read, one slot per expert, so that a
// slot goes from the file to device memory without a device repack. Drop-in for the reference's
// src/model/expert_pack.hpp:1-92: the same file format, byte for byte (a pack written by either side reads in the
// other), and the same names for the format and its host helpers.
//
//   [4 KiB header][zero up to 1 MiB][slot 0][slot 1]...[slot N-1][checksum table: N x {u64 xxh64, u64 present}]
//
// Slot = [w1 codes | w1 scales | w3 codes | w3 scales | w2 codes | w2 scales], each part in the tile-major layout of
// kernels::mx_repack. Slot order: main layers, then the multi-token-prediction stages, each with experts 0..E-1.
// Not here: the checkpoint side (geometry_of, expert_prefix, expert_tensors, config_hash, source_hash), which reads
// safetensors shards; the writer below takes the expert tensors as host arrays and the two fingerprints as values.
#pragma once

#include <cstddef>
#include <cstdint>

namespace unholy::model::pack {

constexpr uint64_t kMagic = 0x3150584c4f48494eull;  // the bytes "NIHOLXP1" read as a little-endian u64
constexpr uint32_t kVersion = 1;
constexpr uint64_t kAlign = 4096;
constexpr uint64_t kHeaderBytes = 4096;
constexpr uint64_t kFirstSlotOffset = uint64_t(1) << 20;
constexpr int kParts = 6;  // w1 codes, w1 scales, w3 codes, w3 scales, w2 codes, w2 scales

// Ref expert_pack.hpp:29-45: the first 4 KiB of the file, the rest of them zero.
struct Header {
  uint64_t magic = kMagic;
  uint32_t version = kVersion;
  uint32_t header_bytes = uint32_t(kHeaderBytes);
  uint32_t n_layers = 0, n_mtp = 0, n_experts = 0, reserved0 = 0;
  uint64_t n_slots = 0;
  uint64_t slot_bytes = 0;
  uint64_t slots_offset = 0;
  uint64_t checksum_offset = 0;  // n_slots x ChecksumEntry
  uint64_t part_offset[kParts] = {};
  uint64_t part_bytes[kParts] = {};
  uint32_t w13_out = 0, w13_in = 0, w2_out = 0, w2_in = 0;  // w1 / w3 [out, in]; w2 [out, in]
  uint64_t config_hash = 0;
  uint64_t source_hash = 0;
  uint64_t reserved[8] = {};
  uint64_t header_hash = 0;  // xxh64 of the bytes before this field
};
static_assert(sizeof(Header) <= kHeaderBytes);
static_assert(offsetof(Header, header_hash) == 256, "the reference's field layout");

struct ChecksumEntry {
  uint64_t hash;
  uint64_t present;
};

// XXH64 (Yann Collet's xxHash, 64-bit variant, as published), seed 0 unless given.
uint64_t xxh64(const void* data, size_t len, uint64_t seed = 0);

inline uint64_t align_up(uint64_t x, uint64_t a = kAlign) { return (x + a - 1) / a * a; }

// Ref expert_pack.hpp:55-62: the slot geometry.
struct Geometry {
  int n_layers = 0, n_mtp = 0, n_experts = 0;
  int w13_out = 0, w13_in = 0, w2_out = 0, w2_in = 0;
  uint64_t part_offset[kParts] = {}, part_bytes[kParts] = {}, slot_bytes = 0;
  size_t n_slots() const { return size_t(n_layers + n_mtp) * n_experts; }
  size_t slot_index(int group, int expert) const { return size_t(group) * n_experts + expert; }
};
// The geometry of experts with w1 / w3 [w13_out, w13_in] and w2 [w2_out, w2_in] (what the reference's geometry_of
// derives from the checkpoint's tensor shapes); throws unless the slot is a multiple of 4096 bytes.
Geometry geometry_for(int n_layers, int n_mtp, int n_experts, int w13_out, int w13_in, int w2_out, int w2_in);
Geometry geometry_from(const Header& h);

// Ref expert_pack.hpp:70-73: one matrix w [n, k/2] + s [n, k/32] to the tile-major layout (tw, ts), and back.
void repack_matrix(const uint8_t* w, const uint8_t* s, uint8_t* tw, uint8_t* ts, int n, int k);
void unrepack_matrix(const uint8_t* tw, const uint8_t* ts, uint8_t* w, uint8_t* s, int n, int k);

// Ref expert_pack.hpp:75-81: file bytes [off, off + len) read as the 4 KiB-aligned superset (for O_DIRECT) into buf
// (4 KiB aligned, aligned_buffer_bytes(len) bytes); returns a pointer to byte `off` inside it.
const uint8_t* read_aligned(int fd, uint64_t off, uint64_t len, uint8_t* buf);
inline size_t aligned_buffer_bytes(uint64_t len) { return size_t(align_up(len) + 2 * kAlign); }
uint8_t* alloc_aligned(size_t bytes);  // 4 KiB aligned; throws
void free_aligned(void* p);

// Ref expert_pack.hpp:88-89: reads and validates a header (magic, version, header hash); throws on a mismatch.
Header read_header(int fd);

// The writer (the reference's tools/expert_pack does this from a checkpoint). parts[slot * 6 + i]: part i of the
// slot's expert in the row-major layout (w [out, in/2] codes, s [out, in/32] e8m0 scales), or all six null for an
// absent slot (written as zeros, present = 0). Writes to path + ".tmp", then renames.
void write_pack(const char* path, const Geometry& g, const uint8_t* const* parts, uint64_t config_hash,
                uint64_t source_hash);

// The loader: slots [first, first + count) of an open pack into device memory at dst (slot i at dst + i * stride,
// stride >= slot_bytes, 256-byte aligned). Eight reader threads, each with two pinned staging buffers of one slot
// taken from a process-wide pool (kept for later calls; at most 16 buffers of the largest slot size loaded), read
// whole slots (or, unverified with fewer slots than threads, 4 KiB-aligned chunks of them), so file reads, checksums
// and host-to-device copies overlap. The checksum table's present flags are always read: an absent slot throws,
// verified or not. With verify, each slot's xxh64 is checked against the table (throws on a mismatch; the first error
// of any thread is the one thrown). Synchronous on `stream` at return.
void load_slots(int fd, const Header& h, size_t first, size_t count, void* dst, size_t stride, bool verify,
                void* stream);

}  // namespace unholy::model::pack
