// Exact-prefix cache: snapshots of every layer's attention state, restored
// on a prefix hit so only the prompt suffix is prefilled.
//
// Mirrors NativeExactPrefixCache and the resident engine's entry pool
// (native/src/native_resident_engine.hip.cpp:121-296 for the cache,
// :553-560 for the pool size, :706-719 for the lookup, :826-836 for the
// restore and :1197-1214 for the capture slot):
//  * a cache entry holds one device allocation with a slot per registered
//    live buffer ("slice"): per-token slices (a full-attention layer's K or V
//    cache, bytes_per_token > 0) store only the prefix's rows, fixed slices
//    (a GDN layer's conv or recurrent state) are stored whole; plus the
//    prompt's terminal hidden row;
//  * the pool has 4 entries up to 32K tokens of capacity, 2 up to 128K, else 1;
//    lookup picks the entry with the longest matching token prefix (first
//    such entry on ties), capture goes to the first empty entry, else to the
//    least recently used one.
// The reference issues one hipMemcpyAsync per slice (80 for the 40-layer
// model); here capture and restore are each one launch of a batched copy
// kernel over a device-side slice table (grid = chunks x slices, 16-byte
// nontemporal loads and stores), so a capture costs one launch however many
// layers are registered.
#include "common.h"

#include <algorithm>
#include <mutex>
#include <new>
#include <vector>

namespace q36 {
namespace {

struct SliceDesc {
  char* live;
  unsigned long long offset;          // byte offset of the slot in an entry
  unsigned long long capacity_bytes;
  unsigned long long bytes_per_token; // 0: fixed slice
};

constexpr unsigned kCopyChunk = 65536;   // bytes per workgroup
constexpr unsigned kCopyThreads = 256;

// blockIdx.y = slice (slice == nslices: the terminal row, capture only),
// blockIdx.x = 64 KiB chunk of that slice's copy.
__global__ __launch_bounds__(kCopyThreads) void prefix_copy_kernel(
    const SliceDesc* __restrict__ table, unsigned nslices, char* snapshot,
    unsigned long long tokens, int to_snapshot, const char* terminal_src,
    unsigned long long terminal_offset, unsigned long long terminal_bytes) {
  const unsigned s = blockIdx.y;
  char* live;
  unsigned long long slot, bytes;
  if (s < nslices) {
    const SliceDesc d = table[s];
    live = d.live;
    slot = d.offset;
    bytes = d.bytes_per_token ? tokens * d.bytes_per_token : d.capacity_bytes;
  } else {
    live = const_cast<char*>(terminal_src);
    slot = terminal_offset;
    bytes = terminal_bytes;
  }
  const unsigned long long c0 = (unsigned long long)blockIdx.x * kCopyChunk;
  if (c0 >= bytes) return;
  const unsigned long long c1 = min(c0 + kCopyChunk, bytes);
  const char* src = to_snapshot ? live : snapshot + slot;
  char* dst = to_snapshot ? snapshot + slot : live;
  // 4 16-byte loads per thread in flight before their stores (measured 4.5%
  // faster than 1, and faster than 2, 8 or 16)
  constexpr unsigned long long kStep = 16ull * kCopyThreads;
  for (unsigned long long i = c0 + 16ull * threadIdx.x; i < c1; i += 4 * kStep) {
    u32x4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (i + u * kStep < c1)
        v[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + i + u * kStep));
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (i + u * kStep < c1)
        __builtin_nontemporal_store(v[u], reinterpret_cast<u32x4*>(dst + i + u * kStep));
  }
}

struct Entry {
  char* snapshot = nullptr;
  std::vector<unsigned> tokens;
  bool valid = false;
  unsigned long long use = 0;
};

struct Pool {
  std::mutex mu;
  int device = 0;
  unsigned max_tokens = 0;
  unsigned long long terminal_bytes = 0;
  unsigned n_entries = 0;
  std::vector<SliceDesc> slices;
  unsigned long long bytes = 0;          // per entry, terminal row included
  unsigned long long terminal_offset = 0;
  SliceDesc* table = nullptr;            // device copy of `slices`
  std::vector<Entry> entries;
  unsigned long long clock = 0;
  bool finalized = false;
};

unsigned matched_prefix(const Entry& e, const unsigned* tokens, unsigned n) {
  if (!e.valid || n < e.tokens.size() ||
      !std::equal(e.tokens.begin(), e.tokens.end(), tokens))
    return 0;
  return (unsigned)e.tokens.size();
}

unsigned long long copy_bytes(const Pool& p, unsigned long long tokens) {
  unsigned long long b = 0;
  for (const SliceDesc& d : p.slices)
    b += d.bytes_per_token ? tokens * d.bytes_per_token : d.capacity_bytes;
  return b;
}

int launch_copy(Pool& p, Entry& e, unsigned long long tokens, bool to_snapshot,
                const void* terminal, void* stream) {
  unsigned long long max_bytes = to_snapshot ? p.terminal_bytes : 0;
  for (const SliceDesc& d : p.slices)
    max_bytes = std::max(max_bytes,
                         d.bytes_per_token ? tokens * d.bytes_per_token : d.capacity_bytes);
  const unsigned chunks = (unsigned)((max_bytes + kCopyChunk - 1) / kCopyChunk);
  const unsigned ny = (unsigned)p.slices.size() + (to_snapshot ? 1u : 0u);
  if (chunks == 0 || ny == 0) return Q36_OK;
  hipLaunchKernelGGL(prefix_copy_kernel, dim3(chunks, ny), dim3(kCopyThreads), 0,
                     static_cast<hipStream_t>(stream), p.table,
                     (unsigned)p.slices.size(), e.snapshot, tokens, to_snapshot ? 1 : 0,
                     static_cast<const char*>(terminal), p.terminal_offset,
                     p.terminal_bytes);
  return static_cast<int>(hipGetLastError());
}

}  // namespace
}  // namespace q36

using namespace q36;

// Pool of exact-prefix cache entries.  entries == 0 picks the reference's
// rule from max_tokens (4 / 2 / 1).  Returns nullptr on bad arguments.
Q36_EXPORT void* qwen36_prefix_cache_create(unsigned max_tokens,
                                            unsigned long long terminal_bytes,
                                            unsigned entries) {
  if (max_tokens == 0 || max_tokens > kMaxTokens || terminal_bytes == 0 ||
      terminal_bytes % 16 != 0 || entries > 16)
    return nullptr;
  Pool* p = new (std::nothrow) Pool();
  if (p == nullptr) return nullptr;
  p->max_tokens = max_tokens;
  p->terminal_bytes = terminal_bytes;
  p->n_entries = entries ? entries : (max_tokens <= 32768u ? 4u : (max_tokens <= 131072u ? 2u : 1u));
  return p;
}

Q36_EXPORT unsigned qwen36_prefix_cache_entries(void* pool) {
  return pool ? static_cast<Pool*>(pool)->n_entries : 0u;
}

// Registers a live device buffer.  bytes_per_token > 0: a per-token slice
// whose capacity must be max_tokens * bytes_per_token; 0: a fixed slice.
// Pointers and sizes must be 16-byte multiples.
Q36_EXPORT int qwen36_prefix_cache_add_slice(void* pool, void* live,
                                             unsigned long long capacity_bytes,
                                             unsigned long long bytes_per_token) {
  Pool* p = static_cast<Pool*>(pool);
  if (p == nullptr || live == nullptr || capacity_bytes == 0 || !aligned16(live) ||
      capacity_bytes % 16 != 0 || bytes_per_token % 16 != 0 ||
      (bytes_per_token != 0 && capacity_bytes != (unsigned long long)p->max_tokens * bytes_per_token))
    return Q36_EINVAL;
  std::lock_guard<std::mutex> lock(p->mu);
  if (p->finalized) return Q36_EINVAL;
  p->slices.push_back(SliceDesc{static_cast<char*>(live), p->bytes, capacity_bytes,
                                bytes_per_token});
  p->bytes += capacity_bytes;
  return Q36_OK;
}

// Allocates, on the current device, every entry's snapshot and the device
// slice table.  Writes the total device bytes to *bytes_out (may be null).
Q36_EXPORT int qwen36_prefix_cache_finalize(void* pool, unsigned long long* bytes_out) {
  Pool* p = static_cast<Pool*>(pool);
  if (p == nullptr) return Q36_EINVAL;
  std::lock_guard<std::mutex> lock(p->mu);
  if (p->finalized || p->slices.empty()) return Q36_EINVAL;
  hipError_t e = hipGetDevice(&p->device);   // entries live on the current device
  if (e != hipSuccess) return (int)e;
  const unsigned long long per_entry = p->bytes + p->terminal_bytes;
  // All-or-nothing: on any failure everything allocated here is freed and
  // the pool is left as it was before the call, so finalize may be retried.
  SliceDesc* table = nullptr;
  std::vector<char*> snaps;
  auto fail = [&](hipError_t err) {
    for (char* q : snaps) (void)hipFree(q);
    if (table != nullptr) (void)hipFree(table);
    (void)hipGetLastError();
    return (int)err;
  };
  e = hipMalloc(reinterpret_cast<void**>(&table), p->slices.size() * sizeof(SliceDesc));
  if (e != hipSuccess) return fail(e);
  e = hipMemcpy(table, p->slices.data(), p->slices.size() * sizeof(SliceDesc),
                hipMemcpyHostToDevice);
  if (e != hipSuccess) return fail(e);
  for (unsigned i = 0; i < p->n_entries; ++i) {
    char* q = nullptr;
    e = hipMalloc(reinterpret_cast<void**>(&q), per_entry);
    if (e != hipSuccess) return fail(e);
    snaps.push_back(q);
  }
  p->terminal_offset = p->bytes;
  p->table = table;
  p->entries.resize(p->n_entries);
  for (unsigned i = 0; i < p->n_entries; ++i) p->entries[i].snapshot = snaps[i];
  p->finalized = true;
  if (bytes_out) *bytes_out = per_entry * p->n_entries;
  return Q36_OK;
}

// Longest stored prefix of tokens[0, n): writes the matched token count and
// the entry index (== entries when nothing matches).
Q36_EXPORT int qwen36_prefix_cache_lookup(void* pool, const unsigned* tokens,
                                          unsigned n, unsigned* matched,
                                          unsigned* index) {
  Pool* p = static_cast<Pool*>(pool);
  if (p == nullptr || matched == nullptr || index == nullptr || (tokens == nullptr && n != 0))
    return Q36_EINVAL;
  std::lock_guard<std::mutex> lock(p->mu);
  unsigned best = 0, best_i = p->n_entries;
  for (unsigned i = 0; i < p->entries.size(); ++i) {
    const unsigned m = matched_prefix(p->entries[i], tokens, n);
    if (m > best) {
      best = m;
      best_i = i;
    }
  }
  *matched = best;
  *index = best_i;
  return Q36_OK;
}

// Copies entry `index` back into the live buffers (per-token slices: its
// stored rows only) on `stream`, marks it most recently used and writes the
// copied bytes to *bytes_out (may be null).
Q36_EXPORT int qwen36_prefix_cache_restore(void* pool, unsigned index, void* stream,
                                           unsigned long long* bytes_out) {
  Pool* p = static_cast<Pool*>(pool);
  if (p == nullptr) return Q36_EINVAL;
  std::lock_guard<std::mutex> lock(p->mu);
  if (!p->finalized || index >= p->entries.size() || !p->entries[index].valid)
    return Q36_EINVAL;
  Entry& e = p->entries[index];
  const int st = launch_copy(*p, e, e.tokens.size(), false, nullptr, stream);
  if (st != Q36_OK) return st;
  e.use = ++p->clock;
  if (bytes_out) *bytes_out = copy_bytes(*p, e.tokens.size());
  return Q36_OK;
}

// Captures the live buffers for the prompt tokens[0, n) and its terminal
// hidden row (terminal_bytes at `terminal`) into the first empty entry, else
// the least recently used one; writes the entry index and copied bytes.
Q36_EXPORT int qwen36_prefix_cache_capture(void* pool, const unsigned* tokens,
                                           unsigned n, const void* terminal,
                                           void* stream, unsigned* index_out,
                                           unsigned long long* bytes_out) {
  Pool* p = static_cast<Pool*>(pool);
  if (p == nullptr || tokens == nullptr || n == 0 || terminal == nullptr ||
      !aligned16(terminal))
    return Q36_EINVAL;
  std::lock_guard<std::mutex> lock(p->mu);
  if (!p->finalized || n > p->max_tokens) return Q36_EINVAL;
  unsigned slot = (unsigned)p->entries.size();
  for (unsigned i = 0; i < p->entries.size(); ++i)
    if (!p->entries[i].valid) {
      slot = i;
      break;
    }
  if (slot == p->entries.size()) {
    slot = 0;
    for (unsigned i = 1; i < p->entries.size(); ++i)
      if (p->entries[i].use < p->entries[slot].use) slot = i;
  }
  Entry& e = p->entries[slot];
  e.valid = false;
  const int st = launch_copy(*p, e, n, true, terminal, stream);
  if (st != Q36_OK) return st;
  e.tokens.assign(tokens, tokens + n);
  e.valid = true;
  e.use = ++p->clock;
  if (index_out) *index_out = slot;
  if (bytes_out) *bytes_out = copy_bytes(*p, n) + p->terminal_bytes;
  return Q36_OK;
}

// Copies entry `index`'s terminal hidden row to `dst` on `stream`.
Q36_EXPORT int qwen36_prefix_cache_copy_terminal(void* pool, unsigned index, void* dst,
                                                 void* stream) {
  Pool* p = static_cast<Pool*>(pool);
  if (p == nullptr || dst == nullptr) return Q36_EINVAL;
  std::lock_guard<std::mutex> lock(p->mu);
  if (!p->finalized || index >= p->entries.size() || !p->entries[index].valid)
    return Q36_EINVAL;
  return (int)hipMemcpyAsync(dst, p->entries[index].snapshot + p->terminal_offset,
                             p->terminal_bytes, hipMemcpyDeviceToDevice,
                             static_cast<hipStream_t>(stream));
}

Q36_EXPORT int qwen36_prefix_cache_destroy(void* pool) {
  Pool* p = static_cast<Pool*>(pool);
  if (p == nullptr) return Q36_EINVAL;
  {
    std::lock_guard<std::mutex> lock(p->mu);
    if (p->finalized || p->table != nullptr) (void)hipSetDevice(p->device);
    for (Entry& e : p->entries)
      if (e.snapshot) (void)hipFree(e.snapshot);
    if (p->table) (void)hipFree(p->table);
  }
  delete p;
  return Q36_OK;
}
