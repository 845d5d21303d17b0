// Host page table of the streaming event cache: (session, first bin) -> device page,
// with a free list and least-recently-used eviction.
//
// The policy is the reference StreamingKVCache's (cortex/cache/streaming.py:133-233):
// a read touches the page (most recently used) and counts a hit, a missing key counts
// a miss; a write reuses the key's page or allocates one -- from the free list (last
// freed first), else by evicting the least recently used page -- and touches it;
// evicting a session frees its pages in the order their keys were first written.
// Here it runs natively, and a whole batch of page writes or window lookups is one
// call: at 256 sessions x 12 pages per window the per-key interpreter work of the
// reference's dict/OrderedDict bookkeeping took longer than the device gather.
//
// Not thread-safe: one caller at a time per table.
#include <stdint.h>

#include <algorithm>
#include <new>
#include <unordered_map>
#include <vector>

#include "common.h"

namespace cortex {
namespace {

struct Key {
  int64_t session, bin;
  bool operator==(const Key& o) const { return session == o.session && bin == o.bin; }
};
struct KeyHash {
  size_t operator()(const Key& k) const {
    uint64_t h = (uint64_t)k.session * 0x9E3779B97F4A7C15ull;
    h ^= (uint64_t)k.bin + 0x7F4A7C159E3779B9ull + (h << 6) + (h >> 2);
    return (size_t)h;
  }
};

struct PageTable {
  int64_t num_pages;
  std::unordered_map<Key, int32_t, KeyHash> table;
  std::vector<Key> key;           // key of each page in use
  std::vector<int64_t> n_events;  // events stored in each page
  std::vector<int64_t> seq;       // first-write order of the page's key
  std::vector<int32_t> prev, next;  // LRU list: head least, tail most recently used
  std::vector<uint8_t> used;
  std::vector<int32_t> free_list;
  int32_t head = -1, tail = -1;
  int64_t hits = 0, misses = 0, in_use = 0, next_seq = 0;

  explicit PageTable(int64_t n)
      : num_pages(n), key(n), n_events(n, 0), seq(n, 0), prev(n, -1), next(n, -1), used(n, 0) {
    free_list.reserve(n);
    for (int64_t p = 0; p < n; ++p) free_list.push_back((int32_t)p);
    table.reserve((size_t)n * 2);
  }

  void unlink(int32_t p) {
    if (prev[p] >= 0) next[prev[p]] = next[p]; else head = next[p];
    if (next[p] >= 0) prev[next[p]] = prev[p]; else tail = prev[p];
    prev[p] = next[p] = -1;
  }
  void push_tail(int32_t p) {
    prev[p] = tail;
    next[p] = -1;
    if (tail >= 0) next[tail] = p; else head = p;
    tail = p;
  }
  void touch(int32_t p) {
    if (tail == p) return;
    unlink(p);
    push_tail(p);
  }
  void free_page(int32_t p) {
    if (used[p]) {
      table.erase(key[p]);
      unlink(p);
      used[p] = 0;
      n_events[p] = 0;
      --in_use;
    }
    free_list.push_back(p);
  }
  int32_t allocate() {
    if (free_list.empty()) free_page(head);  // evict the least recently used page
    const int32_t p = free_list.back();
    free_list.pop_back();
    return p;
  }
  // page of a key (touched, a hit) or -1 (a miss)
  int32_t lookup(const Key& k) {
    auto it = table.find(k);
    if (it == table.end()) {
      ++misses;
      return -1;
    }
    ++hits;
    touch(it->second);
    return it->second;
  }
  int32_t write(const Key& k, int64_t n) {
    int32_t p;
    auto it = table.find(k);
    if (it != table.end()) {
      p = it->second;
    } else {
      p = allocate();
      table.emplace(k, p);
      key[p] = k;
      used[p] = 1;
      seq[p] = next_seq++;
      ++in_use;
      push_tail(p);
    }
    n_events[p] = n;
    touch(p);
    return p;
  }
};

PageTable* as_table(void* h) { return static_cast<PageTable*>(h); }

}  // namespace
}  // namespace cortex

using namespace cortex;

extern "C" {

int cortex_page_table_create(int64_t num_pages, void** out) {
  CORTEX_CHECK_ARG(out != nullptr, "cortex_page_table_create: out must not be null");
  CORTEX_CHECK_ARG(num_pages >= 1 && num_pages <= 0x7fffffffLL, "cortex_page_table_create: num_pages must be in [1, 2^31)");
  PageTable* t = new (std::nothrow) PageTable(num_pages);
  if (!t) {
    set_error("cortex_page_table_create: out of host memory");
    return E_INVALID;
  }
  *out = t;
  return OK;
}

int cortex_page_table_destroy(void* table) {
  delete as_table(table);
  return OK;
}

int cortex_page_table_write(void* table, int64_t n, const int64_t* sessions, const int64_t* bin_starts,
                            const int64_t* n_events, int64_t* page_ids) {
  CORTEX_CHECK_ARG(table && n >= 0, "cortex_page_table_write: null table or negative count");
  if (n == 0) return OK;
  CORTEX_CHECK_ARG(sessions && bin_starts && n_events && page_ids, "cortex_page_table_write: null array");
  PageTable* t = as_table(table);
  for (int64_t i = 0; i < n; ++i) page_ids[i] = t->write(Key{sessions[i], bin_starts[i]}, n_events[i]);
  return OK;
}

int cortex_page_table_lookup(void* table, int64_t session, int64_t bin_start, int64_t* page_id, int64_t* n_events) {
  CORTEX_CHECK_ARG(table && page_id && n_events, "cortex_page_table_lookup: null pointer");
  PageTable* t = as_table(table);
  const int32_t p = t->lookup(Key{session, bin_start});
  *page_id = p;
  *n_events = p >= 0 ? t->n_events[p] : 0;
  return OK;
}

int cortex_page_table_plan(void* table, int64_t n_windows, const int64_t* sessions, const int64_t* window_starts,
                           int64_t window_bins, int64_t bins_per_page, int64_t* items, int64_t items_cap,
                           int64_t* n_items, int64_t* offsets, int64_t* missing_window, int64_t* missing,
                           int64_t* n_missing) {
  CORTEX_CHECK_ARG(table && n_items && offsets && missing_window && n_missing, "cortex_page_table_plan: null pointer");
  CORTEX_CHECK_ARG(n_windows >= 0 && window_bins > 0 && bins_per_page > 0 && window_bins % bins_per_page == 0,
                   "cortex_page_table_plan: window_bins must be a positive multiple of bins_per_page");
  const int64_t per = window_bins / bins_per_page;
  CORTEX_CHECK_ARG(n_windows == 0 || (sessions && window_starts && items && missing),
                   "cortex_page_table_plan: null array");
  CORTEX_CHECK_ARG(items_cap >= n_windows * per, "cortex_page_table_plan: items_cap < n_windows * pages per window");
  PageTable* t = as_table(table);
  int64_t k = 0, row = 0;
  offsets[0] = 0;
  *missing_window = -1;
  *n_missing = 0;
  for (int64_t w = 0; w < n_windows; ++w) {
    const int64_t w0 = window_starts[w];
    CORTEX_CHECK_ARG(w0 % bins_per_page == 0, "cortex_page_table_plan: window start %lld is not a multiple of %lld",
                     (long long)w0, (long long)bins_per_page);
    int64_t nm = 0;
    const int64_t k0 = k;
    for (int64_t j = 0; j < per; ++j) {  // every page of the window is looked up (and counted)
      const int64_t b = w0 + j * bins_per_page;
      const int32_t p = t->lookup(Key{sessions[w], b});
      if (p < 0) {
        missing[nm++] = b;
        continue;
      }
      const int64_t n = t->n_events[p];
      if (n > 0) {
        items[4 * k] = p;
        items[4 * k + 1] = n;
        items[4 * k + 2] = row;
        items[4 * k + 3] = w0;
        ++k;
        row += n;
      }
    }
    if (nm > 0) {  // window w is incomplete: report its missing first bins, plan nothing after it
      *missing_window = w;
      *n_missing = nm;
      *n_items = k0;
      return OK;
    }
    offsets[w + 1] = row;
  }
  *n_items = k;
  return OK;
}

int cortex_page_table_evict_session(void* table, int64_t session, int64_t* freed) {
  CORTEX_CHECK_ARG(table && freed, "cortex_page_table_evict_session: null pointer");
  PageTable* t = as_table(table);
  std::vector<int32_t> pages;
  for (int64_t p = 0; p < t->num_pages; ++p)
    if (t->used[p] && t->key[p].session == session) pages.push_back((int32_t)p);
  // first-written keys first, as a dict iterates its keys
  std::vector<std::pair<int64_t, int32_t>> by_seq;
  by_seq.reserve(pages.size());
  for (int32_t p : pages) by_seq.emplace_back(t->seq[p], p);
  std::sort(by_seq.begin(), by_seq.end());
  for (const auto& sp : by_seq) t->free_page(sp.second);
  *freed = (int64_t)pages.size();
  return OK;
}

int cortex_page_table_stats(void* table, int64_t* hits, int64_t* misses, int64_t* pages_used) {
  CORTEX_CHECK_ARG(table && hits && misses && pages_used, "cortex_page_table_stats: null pointer");
  PageTable* t = as_table(table);
  *hits = t->hits;
  *misses = t->misses;
  *pages_used = t->in_use;
  return OK;
}

}  // extern "C"
