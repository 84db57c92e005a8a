// Host-side paged KV cache: the device page pool, the block table and the page allocator.
//
// Contract of the reference KvCache (include/qwen38/kv_cache.h:19-51): one pool of 64-token pages
// whose ids are shared by every attention layer; a slot's pages are reserved all at once or not at
// all; releasing a slot returns its pages; the device block table is refreshed asynchronously.
//
// Allocator design (this library's own):
//   * free pages are kept as extents (first page -> run length) in an ordered map, and a
//     reservation always takes the lowest free page ids, cutting runs from the front. A fresh pool
//     therefore hands out page 0 first, and sequences get physically contiguous runs of pages
//     whenever the pool is not fragmented (long runs keep a decode wave's loads within one region
//     of HBM, and make page ids predictable in tests);
//   * releasing a slot merges its pages back into the extents (adjacent runs coalesce), so the
//     map's size is bounded by the pool's fragmentation, not by its page count;
//   * the host copy of the block table is the only record of which pages a slot holds: row `slot`
//     lists them in position order and `held[slot]` counts them;
//   * a row only grows between releases, so `synced[slot]` (entries already uploaded) is a
//     watermark: sync() copies entries [synced, held) of each row and nothing else.
// The pool is laid out [layer][page][page_bytes] and zeroed once at creation, so a page never
// holds NaN bit patterns even before its first write.
#include <cstring>
#include <iterator>
#include <map>
#include <new>
#include <vector>

#include "common.hpp"

struct q38a_kv_cache {
  int dtype = Q38A_KV_INT8;
  int kv_heads = 0, layers = 0, num_pages = 0, num_slots = 0, max_pages = 0;
  size_t page_bytes = 0, layer_stride = 0;
  uint8_t* pool = nullptr;
  int32_t* table_dev = nullptr;
  int32_t* table_host = nullptr;  // pinned, [slots][max_pages]
  std::map<int, int> extents;     // free runs: first page -> pages in the run
  int free_count = 0;
  std::vector<int> held;          // pages in each slot's row
  std::vector<int> synced;        // leading entries of each row already on the device

  ~q38a_kv_cache() {
    if (pool) (void)hipFree(pool);
    if (table_dev) (void)hipFree(table_dev);
    if (table_host) (void)hipHostFree(table_host);
  }

  int32_t* row(int slot) { return table_host + size_t(slot) * size_t(max_pages); }
  const int32_t* row(int slot) const { return table_host + size_t(slot) * size_t(max_pages); }

  // Writes `count` of the lowest free page ids to dst (ascending) and removes them from the extents.
  void take_lowest(int count, int32_t* dst) {
    while (count > 0) {
      auto run = extents.begin();
      const int first = run->first, len = run->second;
      const int n = len < count ? len : count;
      for (int i = 0; i < n; ++i) *dst++ = first + i;
      extents.erase(run);
      if (n < len) extents.emplace(first + n, len - n);
      count -= n;
      free_count -= n;
    }
  }

  // Returns one page to the extents, merging it with the runs that end just before / start just
  // after it.
  void give_back(int page) {
    int first = page, len = 1;
    auto next = extents.lower_bound(page);
    if (next != extents.end() && next->first == page + 1) {
      len += next->second;
      next = extents.erase(next);
    }
    if (next != extents.begin()) {
      auto prev = std::prev(next);
      if (prev->first + prev->second == page) {
        first = prev->first;
        len += prev->second;
        extents.erase(prev);
      }
    }
    extents.emplace(first, len);
    ++free_count;
  }
};

using namespace q38a;

extern "C" {

int q38a_kv_cache_create(int dtype, int kv_heads, int layers, int num_pages, int num_slots, int max_pages_per_seq,
                         q38a_kv_cache** out) {
  clear_error();
  if (!out) return set_error(Q38A_ERR_INVALID, "kv_cache_create: out is null");
  *out = nullptr;
  if ((dtype != Q38A_KV_INT8 && dtype != Q38A_KV_BF16 && dtype != Q38A_KV_INT8_VT) || kv_heads <= 0 || layers <= 0 || num_pages <= 0 ||
      num_slots <= 0 || max_pages_per_seq <= 0)
    return set_error(Q38A_ERR_INVALID, "kv_cache_create: bad geometry");
  auto* c = new (std::nothrow) q38a_kv_cache();
  if (!c) return set_error(Q38A_ERR_INVALID, "kv_cache_create: out of host memory");
  c->dtype = dtype;
  c->kv_heads = kv_heads;
  c->layers = layers;
  c->num_pages = num_pages;
  c->num_slots = num_slots;
  c->max_pages = max_pages_per_seq;
  c->page_bytes = q38a_kv_page_bytes(dtype, kv_heads);
  c->layer_stride = c->page_bytes * size_t(num_pages);
  const size_t pool_bytes = c->layer_stride * size_t(layers);
  const size_t table_bytes = size_t(num_slots) * size_t(max_pages_per_seq) * sizeof(int32_t);
  int rc = check_hip(hipMalloc(reinterpret_cast<void**>(&c->pool), pool_bytes), "kv_cache_create: pool");
  if (!rc) rc = check_hip(hipMemset(c->pool, 0, pool_bytes), "kv_cache_create: zero pool");
  if (!rc) rc = check_hip(hipMalloc(reinterpret_cast<void**>(&c->table_dev), table_bytes), "kv_cache_create: table");
  if (!rc) rc = check_hip(hipMemset(c->table_dev, 0, table_bytes), "kv_cache_create: zero table");
  if (!rc) rc = check_hip(hipHostMalloc(reinterpret_cast<void**>(&c->table_host), table_bytes, 0), "kv_cache_create: pinned table");
  if (!rc) rc = check_hip(hipDeviceSynchronize(), "kv_cache_create: sync");
  if (rc) {
    delete c;
    return rc;
  }
  std::memset(c->table_host, 0, table_bytes);
  c->extents.emplace(0, num_pages);  // one run: the whole pool
  c->free_count = num_pages;
  c->held.assign(size_t(num_slots), 0);
  c->synced.assign(size_t(num_slots), 0);
  *out = c;
  return Q38A_OK;
}

void q38a_kv_cache_destroy(q38a_kv_cache* c) { delete c; }

int q38a_kv_cache_desc_get(const q38a_kv_cache* c, q38a_kv_cache_desc* out) {
  clear_error();
  if (!c || !out) return set_error(Q38A_ERR_INVALID, "kv_cache_desc: null argument");
  out->pool = c->pool;
  out->dtype = c->dtype;
  out->kv_heads = c->kv_heads;
  out->num_pages = c->num_pages;
  out->page_bytes = c->page_bytes;
  out->layer_stride = c->layer_stride;
  out->block_table = c->table_dev;
  out->max_pages_per_seq = c->max_pages;
  return Q38A_OK;
}

int q38a_kv_cache_ensure(q38a_kv_cache* c, int slot, int tokens, int* ok) {
  clear_error();
  if (!c || !ok) return set_error(Q38A_ERR_INVALID, "kv_cache_ensure: null argument");
  *ok = 0;
  if (slot < 0 || slot >= c->num_slots) return set_error(Q38A_ERR_INVALID, "kv_cache_ensure: slot %d out of range", slot);
  if (tokens < 0) return set_error(Q38A_ERR_INVALID, "kv_cache_ensure: negative token count");
  const long long want = (static_cast<long long>(tokens) + kPageTokens - 1) / kPageTokens;
  if (want > c->max_pages)
    return set_error(Q38A_ERR_CAPACITY, "kv_cache_ensure: %d tokens need %lld pages; a slot's row has %d", tokens,
                     want, c->max_pages);
  const int have = c->held[size_t(slot)];
  const int missing = int(want) - have;
  if (missing > c->free_count) return Q38A_OK;  // all or nothing: *ok stays 0, nothing changed
  if (missing > 0) {
    c->take_lowest(missing, c->row(slot) + have);
    c->held[size_t(slot)] = int(want);
  }
  *ok = 1;
  return Q38A_OK;
}

int q38a_kv_cache_release(q38a_kv_cache* c, int slot) {
  clear_error();
  if (!c || slot < 0 || slot >= c->num_slots) return set_error(Q38A_ERR_INVALID, "kv_cache_release: bad slot");
  const int32_t* pages = c->row(slot);
  for (int i = 0; i < c->held[size_t(slot)]; ++i) c->give_back(pages[i]);
  c->held[size_t(slot)] = 0;
  c->synced[size_t(slot)] = 0;  // the next reservation rewrites the row from its first entry
  return Q38A_OK;
}

int q38a_kv_cache_sync(q38a_kv_cache* c, void* stream) {
  clear_error();
  if (!c) return set_error(Q38A_ERR_INVALID, "kv_cache_sync: null cache");
  for (int s = 0; s < c->num_slots; ++s) {
    const int from = c->synced[size_t(s)], to = c->held[size_t(s)];
    if (to <= from) continue;
    const size_t at = size_t(s) * size_t(c->max_pages) + size_t(from);
    if (int rc = check_hip(hipMemcpyAsync(c->table_dev + at, c->table_host + at, size_t(to - from) * sizeof(int32_t),
                                          hipMemcpyHostToDevice, static_cast<hipStream_t>(stream)),
                           "kv_cache_sync"))
      return rc;
    c->synced[size_t(s)] = to;
  }
  return Q38A_OK;
}

int q38a_kv_cache_free_pages(const q38a_kv_cache* c) { return c ? c->free_count : -1; }

int q38a_kv_cache_pages_of(const q38a_kv_cache* c, int slot) {
  if (!c || slot < 0 || slot >= c->num_slots) return -1;
  return c->held[size_t(slot)];
}

int q38a_kv_cache_page_list(const q38a_kv_cache* c, int slot, int32_t* pages, int cap, int* n) {
  clear_error();
  if (!c || !n || (cap > 0 && !pages) || slot < 0 || slot >= c->num_slots)
    return set_error(Q38A_ERR_INVALID, "kv_cache_page_list: bad arguments");
  *n = c->held[size_t(slot)];
  const int k = cap < *n ? cap : *n;
  if (k > 0) std::memcpy(pages, c->row(slot), size_t(k) * sizeof(int32_t));
  return Q38A_OK;
}

}  // extern "C"
