// Host-side paged KV cache: the device page pool, the block table and the page free list.
//
// Same contract as the reference KvCache (include/qwen38/kv_cache.h:19-51, src/kv_cache.cpp:14-88):
// one pool of 64-token pages whose ids are shared by every attention layer, pages handed out from
// a free list (page 0 first), ensure() reserves all pages of a request at once or changes
// nothing, release() returns them, and sync() uploads only the block-table rows that changed.
// The pool is laid out [layer][page][page_bytes] and zeroed once at creation, so pages never hold
// NaN bit patterns even before their first write.
#include <cstring>
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
  std::vector<int> free_list;
  std::vector<std::vector<int>> owned;
  std::vector<char> dirty;

  ~q38a_kv_cache() {
    if (pool) (void)hipFree(pool);
    if (table_dev) (void)hipFree(table_dev);
    if (table_host) (void)hipHostFree(table_host);
  }
};

using namespace q38a;

extern "C" {

int q38a_kv_cache_create(int dtype, int kv_heads, int layers, int num_pages, int num_slots, int max_pages_per_seq,
                         q38a_kv_cache** out) {
  clear_error();
  if (!out) return set_error(Q38A_ERR_INVALID, "kv_cache_create: out is null");
  *out = nullptr;
  if ((dtype != Q38A_KV_INT8 && dtype != Q38A_KV_BF16) || kv_heads <= 0 || layers <= 0 || num_pages <= 0 ||
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
  c->free_list.resize(size_t(num_pages));
  for (int i = 0; i < num_pages; ++i) c->free_list[size_t(i)] = num_pages - 1 - i;  // page 0 is handed out first
  c->owned.assign(size_t(num_slots), {});
  c->dirty.assign(size_t(num_slots), 0);
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
  const int need = (tokens + kPageTokens - 1) / kPageTokens;
  if (need > c->max_pages)
    return set_error(Q38A_ERR_CAPACITY, "sequence exceeds the per-sequence context limit (%d tokens)", tokens);
  auto& pages = c->owned[size_t(slot)];
  const int extra = need - int(pages.size());
  if (extra <= 0) {
    *ok = 1;
    return Q38A_OK;
  }
  if (extra > int(c->free_list.size())) return Q38A_OK;  // *ok = 0, nothing changed
  int32_t* row = c->table_host + size_t(slot) * size_t(c->max_pages);
  for (int i = 0; i < extra; ++i) {
    const int page = c->free_list.back();
    c->free_list.pop_back();
    row[pages.size()] = page;
    pages.push_back(page);
  }
  c->dirty[size_t(slot)] = 1;
  *ok = 1;
  return Q38A_OK;
}

int q38a_kv_cache_release(q38a_kv_cache* c, int slot) {
  clear_error();
  if (!c || slot < 0 || slot >= c->num_slots) return set_error(Q38A_ERR_INVALID, "kv_cache_release: bad slot");
  auto& pages = c->owned[size_t(slot)];
  for (auto it = pages.rbegin(); it != pages.rend(); ++it) c->free_list.push_back(*it);
  pages.clear();
  return Q38A_OK;
}

int q38a_kv_cache_sync(q38a_kv_cache* c, void* stream) {
  clear_error();
  if (!c) return set_error(Q38A_ERR_INVALID, "kv_cache_sync: null cache");
  for (int s = 0; s < c->num_slots; ++s) {
    if (!c->dirty[size_t(s)]) continue;
    const size_t off = size_t(s) * size_t(c->max_pages);
    const size_t bytes = c->owned[size_t(s)].size() * sizeof(int32_t);
    if (bytes) {
      if (int rc = check_hip(hipMemcpyAsync(c->table_dev + off, c->table_host + off, bytes, hipMemcpyHostToDevice,
                                            static_cast<hipStream_t>(stream)),
                             "kv_cache_sync"))
        return rc;
    }
    c->dirty[size_t(s)] = 0;
  }
  return Q38A_OK;
}

int q38a_kv_cache_free_pages(const q38a_kv_cache* c) { return c ? int(c->free_list.size()) : -1; }

int q38a_kv_cache_pages_of(const q38a_kv_cache* c, int slot) {
  if (!c || slot < 0 || slot >= c->num_slots) return -1;
  return int(c->owned[size_t(slot)].size());
}

int q38a_kv_cache_page_list(const q38a_kv_cache* c, int slot, int32_t* pages, int cap, int* n) {
  clear_error();
  if (!c || !n || (cap > 0 && !pages) || slot < 0 || slot >= c->num_slots)
    return set_error(Q38A_ERR_INVALID, "kv_cache_page_list: bad arguments");
  const auto& own = c->owned[size_t(slot)];
  *n = int(own.size());
  for (int i = 0; i < cap && i < int(own.size()); ++i) pages[i] = own[size_t(i)];
  return Q38A_OK;
}

}  // extern "C"
