// The expert pack's host side: the format helpers, the writer and the loader (see unholy/model/expert_pack.hpp).
// File format: the reference's src/model/expert_pack.hpp:1-92 and tools/expert_pack/main.cpp:135-142 (slots from
// 1 MiB, the checksum table after them padded to 4 KiB, absent slots {0, 0}).
//
// The loader streams slots through two pinned staging buffers: while slot i's bytes go to the device
// (hipMemcpyAsync on the caller's stream), slot i + 1 is read from the file (pread, O_DIRECT when the file was opened
// with it); with verify, the xxh64 of each staged slot is checked on the host before its copy is issued.
#include <fcntl.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cerrno>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <exception>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>
#include <unordered_map>
#include <utility>
#include <vector>

#include "common.hpp"
#include "unholy/model/expert_pack.hpp"

namespace unholy::model::pack {

namespace {

constexpr size_t kLoadThreads = 8;  // reader threads of load_slots

// Pinned staging buffers of load_slots, kept for the life of the process and reused by later calls (allocating pinned
// memory costs milliseconds per buffer, more than loading a few slots). Portable, so any device can copy from them.
// A buffer is taken by one reader thread at a time and returned only after its last copy has completed. Callers
// request whole-slot buffers (slot bytes + alignment) even for chunked reads, and a request that no free buffer can
// serve first frees the free buffers that are too small: the pool holds at most 2 buffers per reader thread (16) of
// the largest slot size loaded so far, plus any taken at that moment.
class StagingPool {
 public:
  void* take(size_t bytes) {
    std::vector<void*> drop;
    {
      const std::lock_guard<std::mutex> lock(mu_);
      for (size_t i = 0; i < free_.size(); ++i)
        if (free_[i].second >= bytes) {
          void* p = free_[i].first;
          free_.erase(free_.begin() + std::ptrdiff_t(i));
          return p;
        }
      for (const auto& f : free_) {  // every free buffer is smaller than the request
        drop.push_back(f.first);
        size_.erase(f.first);
      }
      free_.clear();
    }
    for (void* d : drop) UH_CHECK(hipHostFree(d));
    void* p = nullptr;
    UH_CHECK(hipHostMalloc(&p, bytes, hipHostMallocPortable));
    const std::lock_guard<std::mutex> lock(mu_);
    size_[p] = bytes;
    return p;
  }
  void give(void* p) {
    const std::lock_guard<std::mutex> lock(mu_);
    free_.emplace_back(p, size_[p]);
  }

 private:
  std::mutex mu_;
  std::vector<std::pair<void*, size_t>> free_;
  std::unordered_map<void*, size_t> size_;
};

StagingPool& staging_pool() {
  static StagingPool* pool = new StagingPool;  // never destroyed: pinned memory is released at process exit
  return *pool;
}

// XXH64 constants and steps as published with xxHash.
constexpr uint64_t kP1 = 0x9E3779B185EBCA87ull, kP2 = 0xC2B2AE3D27D4EB4Full, kP3 = 0x165667B19E3779F9ull,
                   kP4 = 0x85EBCA77C2B2AE63ull, kP5 = 0x27D4EB2F165667C5ull;

constexpr uint64_t rotl64(uint64_t v, int s) { return (v << s) | (v >> (64 - s)); }
uint64_t load_le64(const uint8_t* p) {
  uint64_t v;
  std::memcpy(&v, p, sizeof v);
  return v;
}
uint32_t load_le32(const uint8_t* p) {
  uint32_t v;
  std::memcpy(&v, p, sizeof v);
  return v;
}
// One accumulator lane consuming 8 input bytes.
constexpr uint64_t lane_step(uint64_t acc, uint64_t input) { return rotl64(acc + input * kP2, 31) * kP1; }
// Folding a finished lane into the hash.
constexpr uint64_t fold_lane(uint64_t h, uint64_t lane) { return (h ^ lane_step(0, lane)) * kP1 + kP4; }

void pwrite_all(int fd, const void* data, size_t len, uint64_t off) {
  const uint8_t* p = static_cast<const uint8_t*>(data);
  while (len) {
    const ssize_t n = ::pwrite(fd, p, len, off_t(off));
    if (n < 0) {
      if (errno == EINTR) continue;
      throw std::runtime_error(std::string("expert pack: pwrite: ") + std::strerror(errno));
    }
    p += n;
    off += uint64_t(n);
    len -= size_t(n);
  }
}

}  // namespace

uint64_t xxh64(const void* data, size_t len, uint64_t seed) {
  const uint8_t* p = static_cast<const uint8_t*>(data);
  const uint8_t* const end = p + len;
  uint64_t h;
  if (len >= 32) {
    uint64_t lane[4] = {seed + kP1 + kP2, seed + kP2, seed, seed - kP1};
    for (; end - p >= 32; p += 32)
      for (int i = 0; i < 4; ++i) lane[i] = lane_step(lane[i], load_le64(p + 8 * i));
    h = rotl64(lane[0], 1) + rotl64(lane[1], 7) + rotl64(lane[2], 12) + rotl64(lane[3], 18);
    for (int i = 0; i < 4; ++i) h = fold_lane(h, lane[i]);
  } else {
    h = seed + kP5;
  }
  h += uint64_t(len);
  for (; end - p >= 8; p += 8) h = rotl64(h ^ lane_step(0, load_le64(p)), 27) * kP1 + kP4;
  if (end - p >= 4) {
    h = rotl64(h ^ (uint64_t(load_le32(p)) * kP1), 23) * kP2 + kP3;
    p += 4;
  }
  for (; p < end; ++p) h = rotl64(h ^ (uint64_t(*p) * kP5), 11) * kP1;
  h = (h ^ (h >> 33)) * kP2;
  h = (h ^ (h >> 29)) * kP3;
  return h ^ (h >> 32);
}

Geometry geometry_for(int n_layers, int n_mtp, int n_experts, int w13_out, int w13_in, int w2_out, int w2_in) {
  if (n_layers < 0 || n_mtp < 0 || n_experts <= 0 || n_layers + n_mtp <= 0)
    throw std::runtime_error("expert pack: no slots");
  for (const int d : {w13_out, w2_out})
    if (d <= 0 || d % 16) throw std::runtime_error("expert pack: output width % 16");
  for (const int d : {w13_in, w2_in})
    if (d <= 0 || d % 64) throw std::runtime_error("expert pack: input width % 64");
  Geometry g;
  g.n_layers = n_layers;
  g.n_mtp = n_mtp;
  g.n_experts = n_experts;
  g.w13_out = w13_out;
  g.w13_in = w13_in;
  g.w2_out = w2_out;
  g.w2_in = w2_in;
  const uint64_t codes13 = uint64_t(w13_out) * w13_in / 2, scales13 = uint64_t(w13_out) * w13_in / 32;
  const uint64_t codes2 = uint64_t(w2_out) * w2_in / 2, scales2 = uint64_t(w2_out) * w2_in / 32;
  const uint64_t bytes[kParts] = {codes13, scales13, codes13, scales13, codes2, scales2};
  for (int i = 0; i < kParts; ++i) {
    g.part_offset[i] = g.slot_bytes;
    g.part_bytes[i] = bytes[i];
    g.slot_bytes += bytes[i];
  }
  if (g.slot_bytes % kAlign) throw std::runtime_error("expert pack: slot size is not a multiple of 4096");
  return g;
}

Geometry geometry_from(const Header& h) {
  Geometry g;
  g.n_layers = int(h.n_layers);
  g.n_mtp = int(h.n_mtp);
  g.n_experts = int(h.n_experts);
  g.w13_out = int(h.w13_out);
  g.w13_in = int(h.w13_in);
  g.w2_out = int(h.w2_out);
  g.w2_in = int(h.w2_in);
  for (int i = 0; i < kParts; ++i) {
    g.part_offset[i] = h.part_offset[i];
    g.part_bytes[i] = h.part_bytes[i];
  }
  g.slot_bytes = h.slot_bytes;
  return g;
}

// The tile-major layout (16-output tiles of 64-input slabs): row r's 32-byte run j goes to chunk j * (n / 16) + r / 16
// at (r % 16) * 32; its scale b (of 32 inputs) to chunk b / 2 at (r % 16) * 2 + b % 2.
void repack_matrix(const uint8_t* w, const uint8_t* s, uint8_t* tw, uint8_t* ts, int n, int k) {
  const size_t tiles = size_t(n) / 16, runs = size_t(k) / 64, blocks = size_t(k) / 32;
  for (size_t r = 0; r < size_t(n); ++r) {
    const size_t tile = r / 16, lane = r % 16;
    for (size_t j = 0; j < runs; ++j)
      std::memcpy(tw + (j * tiles + tile) * 512 + lane * 32, w + r * (size_t(k) / 2) + j * 32, 32);
    for (size_t b = 0; b < blocks; ++b) ts[((b / 2) * tiles + tile) * 32 + lane * 2 + b % 2] = s[r * blocks + b];
  }
}
void unrepack_matrix(const uint8_t* tw, const uint8_t* ts, uint8_t* w, uint8_t* s, int n, int k) {
  const size_t tiles = size_t(n) / 16, runs = size_t(k) / 64, blocks = size_t(k) / 32;
  for (size_t r = 0; r < size_t(n); ++r) {
    const size_t tile = r / 16, lane = r % 16;
    for (size_t j = 0; j < runs; ++j)
      std::memcpy(w + r * (size_t(k) / 2) + j * 32, tw + (j * tiles + tile) * 512 + lane * 32, 32);
    for (size_t b = 0; b < blocks; ++b) s[r * blocks + b] = ts[((b / 2) * tiles + tile) * 32 + lane * 2 + b % 2];
  }
}

const uint8_t* read_aligned(int fd, uint64_t off, uint64_t len, uint8_t* buf) {
  const uint64_t first = off / kAlign * kAlign, last = align_up(off + len);
  uint64_t got = 0;
  while (got < last - first) {
    const ssize_t n = ::pread(fd, buf + got, size_t(last - first - got), off_t(first + got));
    if (n < 0) {
      if (errno == EINTR) continue;
      throw std::runtime_error(std::string("expert pack: pread: ") + std::strerror(errno));
    }
    if (n == 0) break;  // end of file inside the aligned tail
    got += uint64_t(n);
  }
  if (got < off + len - first) throw std::runtime_error("expert pack: short read");
  return buf + (off - first);
}

uint8_t* alloc_aligned(size_t bytes) {
  void* p = nullptr;
  if (posix_memalign(&p, kAlign, bytes ? bytes : kAlign)) throw std::runtime_error("expert pack: out of memory");
  return static_cast<uint8_t*>(p);
}
void free_aligned(void* p) { std::free(p); }

Header read_header(int fd) {
  uint8_t* buf = alloc_aligned(aligned_buffer_bytes(kHeaderBytes));
  Header h;
  try {
    std::memcpy(&h, read_aligned(fd, 0, kHeaderBytes, buf), sizeof h);
  } catch (...) {
    free_aligned(buf);
    throw;
  }
  free_aligned(buf);
  if (h.magic != kMagic) throw std::runtime_error("expert pack: bad magic");
  if (h.version != kVersion) throw std::runtime_error("expert pack: unsupported version");
  if (h.header_hash != xxh64(&h, offsetof(Header, header_hash))) throw std::runtime_error("expert pack: header hash");
  return h;
}

void write_pack(const char* path, const Geometry& g, const uint8_t* const* parts, uint64_t config_hash,
                uint64_t source_hash) {
  if (!path || !parts) throw std::runtime_error("expert pack: null argument");
  const size_t n = g.n_slots();
  Header h;
  h.n_layers = uint32_t(g.n_layers);
  h.n_mtp = uint32_t(g.n_mtp);
  h.n_experts = uint32_t(g.n_experts);
  h.n_slots = n;
  h.slot_bytes = g.slot_bytes;
  h.slots_offset = kFirstSlotOffset;
  h.checksum_offset = kFirstSlotOffset + n * g.slot_bytes;
  for (int i = 0; i < kParts; ++i) {
    h.part_offset[i] = g.part_offset[i];
    h.part_bytes[i] = g.part_bytes[i];
  }
  h.w13_out = uint32_t(g.w13_out);
  h.w13_in = uint32_t(g.w13_in);
  h.w2_out = uint32_t(g.w2_out);
  h.w2_in = uint32_t(g.w2_in);
  h.config_hash = config_hash;
  h.source_hash = source_hash;
  h.header_hash = xxh64(&h, offsetof(Header, header_hash));

  const std::string tmp = std::string(path) + ".tmp";
  const int fd = ::open(tmp.c_str(), O_WRONLY | O_CREAT | O_TRUNC, 0644);
  if (fd < 0) throw std::runtime_error("expert pack: cannot create " + tmp + ": " + std::strerror(errno));
  uint8_t* slot = nullptr;
  try {
    std::vector<uint8_t> head(kFirstSlotOffset, 0);
    std::memcpy(head.data(), &h, sizeof h);
    pwrite_all(fd, head.data(), head.size(), 0);
    slot = alloc_aligned(g.slot_bytes);
    std::vector<ChecksumEntry> table(n, ChecksumEntry{0, 0});
    for (size_t i = 0; i < n; ++i) {
      const uint8_t* const* p = parts + i * kParts;
      const bool present = p[0] != nullptr;
      std::memset(slot, 0, g.slot_bytes);
      if (present) {
        for (int m = 0; m < 3; ++m) {  // w1, w3, w2
          const int rows = m < 2 ? g.w13_out : g.w2_out, cols = m < 2 ? g.w13_in : g.w2_in;
          if (!p[2 * m] || !p[2 * m + 1]) throw std::runtime_error("expert pack: a present slot with a null part");
          repack_matrix(p[2 * m], p[2 * m + 1], slot + g.part_offset[2 * m], slot + g.part_offset[2 * m + 1], rows,
                        cols);
        }
        table[i] = ChecksumEntry{xxh64(slot, g.slot_bytes), 1};
      }
      pwrite_all(fd, slot, g.slot_bytes, kFirstSlotOffset + i * g.slot_bytes);
    }
    std::vector<uint8_t> tbytes(align_up(n * sizeof(ChecksumEntry)), 0);
    std::memcpy(tbytes.data(), table.data(), n * sizeof(ChecksumEntry));
    pwrite_all(fd, tbytes.data(), tbytes.size(), h.checksum_offset);
  } catch (...) {
    free_aligned(slot);
    ::close(fd);
    ::unlink(tmp.c_str());
    throw;
  }
  free_aligned(slot);
  if (::close(fd)) throw std::runtime_error("expert pack: close failed");
  if (std::rename(tmp.c_str(), path)) throw std::runtime_error(std::string("expert pack: rename: ") + std::strerror(errno));
}

void load_slots(int fd, const Header& h, size_t first, size_t count, void* dst, size_t stride, bool verify,
                void* stream) {
  if (first + count > h.n_slots) throw std::runtime_error("expert pack: slot range past the pack");
  if (!dst || stride < h.slot_bytes || stride % 256) throw std::runtime_error("expert pack: destination stride");
  if (count == 0) return;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  // The checksum table is read for every load (n_slots entries, a few KiB): its present flags refuse an absent slot
  // whether or not the slots are verified (an absent slot's bytes are zeros, not an expert).
  std::vector<ChecksumEntry> table;
  {
    const size_t tb = h.n_slots * sizeof(ChecksumEntry);
    uint8_t* buf = alloc_aligned(aligned_buffer_bytes(tb));
    table.resize(h.n_slots);
    try {
      std::memcpy(table.data(), read_aligned(fd, h.checksum_offset, tb, buf), tb);
    } catch (...) {
      free_aligned(buf);
      throw;
    }
    free_aligned(buf);
  }
  for (size_t i = 0; i < count; ++i)
    if (!table[first + i].present)
      throw std::runtime_error("expert pack: slot " + std::to_string(first + i) + " is absent");
  // Reader threads, as the reference's stream test issues whole-slot reads from several threads: each thread claims
  // slots from a shared counter and owns two pinned staging buffers (4 KiB aligned for O_DIRECT; slots start on
  // 4 KiB boundaries and are whole 4 KiB multiples, so each read is exactly its slot). A thread's file read and
  // checksum of one slot overlap the host-to-device copy of its previous one and the other threads' work.
  int device = 0;
  UH_CHECK(hipGetDevice(&device));
  // Fewer unverified slots than threads: each slot is read as nch 4 KiB-aligned chunks (work items), so every thread
  // has work. A verified slot stays whole: its XXH64 runs over it in order.
  const size_t want = (!verify && count < kLoadThreads) ? (kLoadThreads + count - 1) / count : 1;
  const uint64_t cb = want > 1 ? align_up((h.slot_bytes + want - 1) / want) : h.slot_bytes;
  const size_t nch = size_t((h.slot_bytes + cb - 1) / cb), items = count * nch;
  const int nthreads = int(std::min<size_t>(items, kLoadThreads));
  std::atomic<size_t> next{0};
  std::atomic<bool> failed{false};
  std::mutex err_mu;
  std::exception_ptr err;
  // O_DIRECT reads cannot target the pinned staging (the kernel cannot pin those pages for the transfer: pread fails
  // with EFAULT), so with an O_DIRECT descriptor each reader reads into an ordinary aligned buffer and copies from it.
  const int fl = fcntl(fd, F_GETFL);
  const bool direct = fl != -1 && (fl & O_DIRECT) != 0;
  const auto reader = [&] {
    void* stage[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    uint8_t* bounce = nullptr;
    try {
      if (direct) bounce = alloc_aligned(aligned_buffer_bytes(cb));
      UH_CHECK(hipSetDevice(device));
      for (int b = 0; b < 2; ++b) {
        stage[b] = staging_pool().take(h.slot_bytes + kAlign);  // whole-slot size: chunked reads reuse them
        UH_CHECK(hipEventCreateWithFlags(&done[b], hipEventDisableTiming));
      }
      for (int n = 0; !failed.load(std::memory_order_relaxed); ++n) {
        const size_t item = next.fetch_add(1);
        if (item >= items) break;
        const size_t i = item / nch, c = item % nch;
        const uint64_t len = std::min<uint64_t>(cb, h.slot_bytes - c * cb);
        const uint64_t off = h.slots_offset + (first + i) * h.slot_bytes + c * cb;
        const int b = n & 1;
        UH_CHECK(hipEventSynchronize(done[b]));  // the copy that last used this buffer is over
        uint8_t* a = reinterpret_cast<uint8_t*>(align_up(reinterpret_cast<uintptr_t>(stage[b])));
        if (direct)
          std::memcpy(a, read_aligned(fd, off, len, bounce), len);
        else
          read_aligned(fd, off, len, a);
        if (verify) {  // nch == 1: the whole slot
          const ChecksumEntry& e = table[first + i];
          if (xxh64(a, h.slot_bytes) != e.hash)
            throw std::runtime_error("expert pack: slot " + std::to_string(first + i) + " checksum mismatch");
        }
        UH_CHECK(hipMemcpyAsync(static_cast<uint8_t*>(dst) + i * stride + c * cb, a, len, hipMemcpyHostToDevice, st));
        UH_CHECK(hipEventRecord(done[b], st));
      }
    } catch (...) {
      failed = true;
      const std::lock_guard<std::mutex> lock(err_mu);
      if (!err) err = std::current_exception();
    }
    if (bounce) free_aligned(bounce);
    for (int b = 0; b < 2; ++b) {  // a buffer is freed only once its copy is over
      if (done[b]) (void)hipEventSynchronize(done[b]), (void)hipEventDestroy(done[b]);
      if (stage[b]) staging_pool().give(stage[b]);
    }
  };
  std::vector<std::thread> pool;
  for (int t = 1; t < nthreads; ++t) pool.emplace_back(reader);
  reader();
  for (auto& th : pool) th.join();
  if (err) std::rethrow_exception(err);
  UH_CHECK(hipStreamSynchronize(st));
}

}  // namespace unholy::model::pack
