// The C ABI of libquail_host.so (include/quail_host.h): status codes and the
// per-thread error message around the host library's classes.
#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <new>
#include <stdexcept>

#include "../../include/quail_host.h"
#include "host.h"

using namespace qp;

namespace {

thread_local char g_error[512] = "";

void set_error(const char* msg) { snprintf(g_error, sizeof(g_error), "%s", msg); }

// Run f; turn a library Error (or an allocation failure) into a status.
template <class F>
int64_t guarded(F&& f) {
  try {
    return f();
  } catch (const Error& e) {
    set_error(e.message.c_str());
    return e.code;
  } catch (const std::bad_alloc&) {
    set_error("host library: out of memory");
    return kStateError;
  } catch (const std::out_of_range&) {
    set_error("host library: index out of range");
    return kValueError;
  }
}

template <class T>
T* as(void* p, const char* what) {
  if (!p) fail(kValueError, "%s: null handle", what);
  return static_cast<T*>(p);
}

template <class T>
const T* as(const void* p, const char* what) {
  if (!p) fail(kValueError, "%s: null handle", what);
  return static_cast<const T*>(p);
}

int64_t copy_out(const std::vector<int32_t>& v, int32_t* out, int64_t cap) {
  if (out && (int64_t)v.size() <= cap) std::copy(v.begin(), v.end(), out);
  return (int64_t)v.size();
}

int64_t copy_out(const std::vector<int64_t>& v, int64_t* out, int64_t cap) {
  if (out && (int64_t)v.size() <= cap) std::copy(v.begin(), v.end(), out);
  return (int64_t)v.size();
}

}  // namespace

extern "C" {

int qp_version(void) { return 1; }
const char* qp_last_error(void) { return g_error; }

// ---- arena -------------------------------------------------------------------

void* qp_arena_new(int32_t n_pages, int32_t page_tokens) {
  try {
    return new Arena(n_pages, page_tokens);
  } catch (const Error& e) {
    set_error(e.message.c_str());
  } catch (const std::bad_alloc&) {
    set_error("arena: out of memory");
  }
  return nullptr;
}

void qp_arena_delete(void* arena) { delete static_cast<Arena*>(arena); }

int qp_arena_stats(const void* arena, int64_t* out) {
  return (int)guarded([&] {
    const Arena* a = as<Arena>(arena, "arena");
    out[0] = a->n_pages();
    out[1] = a->page_tokens();
    out[2] = a->free_pages();
    out[3] = a->retained_pages();
    out[4] = a->resident_tokens();
    out[5] = a->retained_prefix_tokens();
    out[6] = (int64_t)a->resident_keys().size();
    out[7] = a->evicted_keys;
    out[8] = a->evicted_pages;
    out[9] = a->evicted_prefix_tokens;
    out[10] = a->retention_cap;
    out[11] = (int64_t)a->retained_keys().size();
    for (int i = 12; i < 16; ++i) out[i] = 0;
    return (int64_t)kOk;
  });
}

int64_t qp_arena_free_list(const void* arena, int32_t* out, int64_t cap) {
  return guarded([&] { return copy_out(as<Arena>(arena, "arena")->free_stack(), out, cap); });
}

int qp_arena_is_resident(const void* arena, int64_t key) {
  return (int)guarded([&] { return (int64_t)as<Arena>(arena, "arena")->resident(key); });
}

int qp_arena_key_info(const void* arena, int64_t key, int64_t* out) {
  return (int)guarded([&] {
    const KeyState& s = as<Arena>(arena, "arena")->state(key);
    out[0] = s.tokens;
    out[1] = s.n_borrowed;
    out[2] = (int64_t)s.pages.size();
    out[3] = s.pinned;
    out[4] = s.retained;
    out[5] = s.retained_tokens;
    out[6] = s.queued;
    out[7] = s.deferred;
    return (int64_t)kOk;
  });
}

int64_t qp_arena_table(const void* arena, int64_t key, int32_t* out, int64_t cap) {
  return guarded([&] { return copy_out(as<Arena>(arena, "arena")->state(key).pages, out, cap); });
}

int qp_arena_alloc(void* arena, int64_t key, int64_t tokens, int64_t capacity,
                   const int32_t* borrowed, int32_t n_borrowed) {
  return (int)guarded([&] {
    return (int64_t)(as<Arena>(arena, "arena")->alloc(key, tokens, capacity, borrowed, n_borrowed)
                         ? kOk : kNone);
  });
}

int64_t qp_arena_shared_pages(const void* arena, int64_t parent, int64_t shared, int64_t start,
                              int32_t* out, int64_t cap) {
  return guarded([&] {
    return copy_out(as<Arena>(arena, "arena")->shared_pages(parent, shared, start), out, cap);
  });
}

int64_t qp_arena_release_pages(void* arena, const int32_t* pages, int64_t n) {
  return guarded([&] {
    Arena* a = as<Arena>(arena, "arena");
    for (int64_t i = 0; i < n; ++i)
      if (pages[i] < 0 || pages[i] >= a->n_pages()) fail(kValueError, "page %d", pages[i]);
    return (int64_t)a->release_pages(pages, (size_t)n);
  });
}

int64_t qp_arena_free_now(void* arena, int64_t key) {
  return guarded([&] { return (int64_t)as<Arena>(arena, "arena")->free_now(key); });
}

int64_t qp_arena_drop_leading(void* arena, int64_t key, int64_t pages) {
  return guarded([&] { return (int64_t)as<Arena>(arena, "arena")->drop_leading(key, pages); });
}

int64_t qp_arena_rewind(void* arena, int64_t key, int64_t tokens) {
  return guarded([&] { return (int64_t)as<Arena>(arena, "arena")->rewind(key, tokens); });
}

int qp_arena_grow(void* arena, int64_t key, int64_t capacity, int64_t* added) {
  return (int)guarded([&] {
    const int64_t n = as<Arena>(arena, "arena")->grow(key, capacity);
    if (n < 0) return (int64_t)kNone;
    *added = n;
    return (int64_t)kOk;
  });
}

int qp_arena_pin(void* arena, int64_t key) {
  return (int)guarded([&] {
    as<Arena>(arena, "arena")->pin(key);
    return (int64_t)kOk;
  });
}

int64_t qp_arena_sole_pages(const void* arena, int64_t key) {
  return guarded([&] { return as<Arena>(arena, "arena")->sole_pages(key); });
}

int qp_arena_retain(void* arena, int64_t key, const double* priority, int32_t n_priority) {
  return (int)guarded([&] {
    if (n_priority < 0) fail(kValueError, "priority of %d values", (int)n_priority);
    Priority p;
    if (priority) p.v.assign(priority, priority + n_priority);
    as<Arena>(arena, "arena")->retain(key, priority ? &p : nullptr);
    return (int64_t)kOk;
  });
}

int qp_arena_pop_victim(void* arena, const int64_t* keep, int64_t n_keep, int64_t* out) {
  return (int)guarded([&] {
    std::vector<int64_t> k(keep, keep + (keep ? n_keep : 0));
    return (int64_t)(as<Arena>(arena, "arena")->pop_victim(k, &out[0], &out[1], &out[2]) ? kOk
                                                                                         : kNone);
  });
}

int qp_arena_clear_retention(void* arena) {
  return (int)guarded([&] {
    as<Arena>(arena, "arena")->clear_retention_heap();
    return (int64_t)kOk;
  });
}

int64_t qp_arena_retained_keys(const void* arena, int64_t* out, int64_t cap) {
  return guarded([&] { return copy_out(as<Arena>(arena, "arena")->retained_keys(), out, cap); });
}

int64_t qp_arena_resident_keys(const void* arena, int64_t* out, int64_t cap) {
  return guarded([&] { return copy_out(as<Arena>(arena, "arena")->resident_keys(), out, cap); });
}

int qp_arena_set_retention_cap(void* arena, int64_t cap_pages) {
  return (int)guarded([&] {
    as<Arena>(arena, "arena")->retention_cap = cap_pages;
    return (int64_t)kOk;
  });
}

int qp_arena_activate(void* arena, int64_t key, int64_t tokens, int64_t capacity, int64_t parent,
                      int64_t shared) {
  return (int)guarded([&] {
    return (int64_t)(as<Arena>(arena, "arena")->activate(key, tokens, capacity, parent, shared)
                         ? kOk : kNone);
  });
}

int qp_arena_alloc_temporary(void* arena, int64_t tokens, int64_t* key) {
  return (int)guarded([&] {
    const int64_t k = as<Arena>(arena, "arena")->alloc_temporary(tokens);
    if (k == 0) return (int64_t)kNone;
    *key = k;
    return (int64_t)kOk;
  });
}

int qp_arena_hold(void* arena, int64_t key, int64_t borrowers) {
  return (int)guarded([&] {
    as<Arena>(arena, "arena")->hold(key, borrowers);
    return (int64_t)kOk;
  });
}

int qp_arena_release(void* arena, int64_t key) {
  return (int)guarded([&] {
    as<Arena>(arena, "arena")->release(key);
    return (int64_t)kOk;
  });
}

int qp_arena_drop_holds(void* arena, const int64_t* keys, int64_t n, int32_t all) {
  return (int)guarded([&] {
    return (int64_t)as<Arena>(arena, "arena")->drop_holds(keys, (size_t)(keys ? n : 0), all != 0);
  });
}

int qp_arena_held(const void* arena, int64_t key) {
  return (int)guarded([&] { return (int64_t)as<Arena>(arena, "arena")->held(key); });
}

int64_t qp_arena_free_key(void* arena, int64_t key) {
  return guarded([&] { return (int64_t)as<Arena>(arena, "arena")->free_key(key); });
}

int64_t qp_arena_evict_key(void* arena, int64_t key) {
  return guarded([&] { return (int64_t)as<Arena>(arena, "arena")->evict_key(key); });
}

int64_t qp_arena_evict_retained(void* arena, int64_t pages_needed) {
  return guarded([&] { return as<Arena>(arena, "arena")->evict_retained(pages_needed); });
}

int64_t qp_arena_drain_evictions(void* arena, int64_t* keys, int64_t* tokens, int64_t* pages,
                                 int64_t cap) {
  return guarded([&] {
    Arena* a = as<Arena>(arena, "arena");
    const int64_t n = std::min<int64_t>(cap, (int64_t)a->events.size());
    for (int64_t i = 0; i < n; ++i) {
      keys[i] = a->events[i].key;
      tokens[i] = a->events[i].tokens;
      pages[i] = a->events[i].pages;
    }
    a->events.erase(a->events.begin(), a->events.begin() + n);
    return n;
  });
}

// ---- token tables --------------------------------------------------------------

void* qp_tokens_new(void) { return new (std::nothrow) TokenTable(); }
void qp_tokens_delete(void* tokens) { delete static_cast<TokenTable*>(tokens); }

int64_t qp_tokens_add(void* tokens, const void* const* data, const int64_t* lens,
                      const int32_t* elem_bytes, int32_t n_parts) {
  return guarded([&] {
    std::vector<TokenPart> parts(n_parts);
    for (int32_t i = 0; i < n_parts; ++i) parts[i] = TokenPart{data[i], lens[i], elem_bytes[i]};
    return as<TokenTable>(tokens, "tokens")->add(parts.data(), n_parts);
  });
}

int64_t qp_tokens_add_flat(void* tokens, const void* data, int32_t elem_bytes, int64_t n,
                           const int64_t* offsets) {
  return guarded([&] {
    TokenTable* t = as<TokenTable>(tokens, "tokens");
    if (n < 0 || (n > 0 && !offsets)) fail(kValueError, "add_flat: %lld entries", (long long)n);
    int64_t first = t->size();
    for (int64_t i = 0; i < n; ++i) {
      if (offsets[i + 1] < offsets[i]) fail(kValueError, "add_flat: offsets decrease at %lld", (long long)i);
      const TokenPart part{static_cast<const char*>(data) + offsets[i] * elem_bytes,
                           offsets[i + 1] - offsets[i], elem_bytes};
      t->add(&part, 1);
    }
    return first;
  });
}

int64_t qp_tokens_length(const void* tokens, int64_t entry) {
  return guarded([&] {
    const TokenTable* t = as<TokenTable>(tokens, "tokens");
    if (entry < 0 || entry >= t->size()) fail(kValueError, "token entry %lld", (long long)entry);
    return t->length(entry);
  });
}

int qp_prefix_tree(const void* ids, int32_t elem_bytes, int64_t n, const int64_t* offsets,
                   int64_t page_tokens, int64_t* order, int64_t* parent, int64_t* shared) {
  return (int)guarded([&] {
    prefix_tree(ids, elem_bytes, n, offsets, page_tokens, order, parent, shared);
    return (int64_t)kOk;
  });
}

// ---- chunk builder -------------------------------------------------------------

void* qp_chunk_new(void) { return new (std::nothrow) ChunkBuilder(); }
void qp_chunk_delete(void* chunk) { delete static_cast<ChunkBuilder*>(chunk); }

int qp_chunk_reset(void* chunk) {
  return (int)guarded([&] {
    as<ChunkBuilder>(chunk, "chunk")->reset();
    return (int64_t)kOk;
  });
}

int qp_chunk_add_group(void* chunk, int64_t key, int64_t read_key, int32_t has_read, int32_t fresh,
                       int64_t start, int64_t f, int64_t write_suffix_tokens,
                       const void* prefix_src, int64_t prefix_entry, int64_t prefix_skip,
                       const void* suffix_src, const int32_t* suffix_entries, int32_t n_suffix) {
  return (int)guarded([&] {
    if (fresh && !prefix_src) fail(kValueError, "a fresh group needs its prefix tokens");
    if (n_suffix && (!suffix_src || !suffix_entries)) fail(kValueError, "suffixes without tokens");
    if (n_suffix < 0 || start < 0 || f < 0 || write_suffix_tokens < 0 || prefix_skip < 0)
      fail(kValueError, "negative group field");
    GroupSpec g{};
    g.key = key;
    g.read_key = read_key;
    g.has_read = has_read != 0;
    g.fresh = fresh != 0;
    g.start = start;
    g.f = f;
    g.write_suffix_tokens = write_suffix_tokens;
    g.prefix_src = static_cast<const TokenTable*>(prefix_src);
    g.prefix_entry = prefix_entry;
    g.prefix_skip = prefix_skip;
    g.suffix_src = static_cast<const TokenTable*>(suffix_src);
    as<ChunkBuilder>(chunk, "chunk")->add_group(g, suffix_entries, n_suffix);
    return (int64_t)kOk;
  });
}

int qp_chunk_build(void* chunk, void* arena, int32_t tree_path) {
  return (int)guarded([&] {
    as<ChunkBuilder>(chunk, "chunk")->build(*as<Arena>(arena, "arena"), tree_path != 0);
    return (int64_t)kOk;
  });
}

int qp_chunk_summary(const void* chunk, int64_t* out) {
  return (int)guarded([&] {
    const ChunkBuilder* b = as<ChunkBuilder>(chunk, "chunk");
    const int64_t v[16] = {b->tokens, b->max_a, b->has_reads, b->reads_max_q, b->reads_max_used,
                           b->reads_rows, b->has_unified, b->uni_max_q, b->uni_max_used,
                           b->own_pairs, b->unified_pairs, b->unified_kv_rows, b->read_pairs,
                           b->read_kv_rows, (int64_t)b->temporaries.size(),
                           (int64_t)b->fresh_keys.size()};
    std::copy(v, v + 16, out);
    return (int64_t)kOk;
  });
}

int qp_chunk_arrays(const void* chunk, int64_t* out) {
  return (int)guarded([&] {
    const ChunkBuilder* b = as<ChunkBuilder>(chunk, "chunk");
    for (int i = 0; i < kNumArrays; ++i) {
      const auto& a = b->arrays[i];
      out[4 * i] = a.present;
      out[4 * i + 1] = a.wide ? (int64_t)a.i64.size() : (int64_t)a.i32.size();
      out[4 * i + 2] = a.rows;
      out[4 * i + 3] = a.cols;
    }
    return (int64_t)kOk;
  });
}

int64_t qp_chunk_emit(const void* chunk, void* dst, int64_t cap, int64_t* offsets) {
  return guarded([&] {
    const ChunkBuilder* b = as<ChunkBuilder>(chunk, "chunk");
    int64_t total = 0;
    for (int i = 0; i < kNumArrays; ++i) {
      const auto& a = b->arrays[i];
      if (!a.present) {
        offsets[i] = -1;
        continue;
      }
      offsets[i] = total;
      total += (a.bytes() + 15) / 16 * 16;
    }
    if (dst == nullptr) return total;
    if (cap < total) fail(kValueError, "chunk staging needs %lld bytes, %lld given", (long long)total,
                          (long long)cap);
    for (int i = 0; i < kNumArrays; ++i) {
      const auto& a = b->arrays[i];
      if (a.present && a.bytes()) std::memcpy(static_cast<char*>(dst) + offsets[i], a.data(), a.bytes());
    }
    return total;
  });
}

int64_t qp_chunk_temporaries(const void* chunk, int64_t* out, int64_t cap) {
  return guarded([&] { return copy_out(as<ChunkBuilder>(chunk, "chunk")->temporaries, out, cap); });
}

int64_t qp_chunk_fresh_keys(const void* chunk, int64_t* out, int64_t cap) {
  return guarded([&] { return copy_out(as<ChunkBuilder>(chunk, "chunk")->fresh_keys, out, cap); });
}

// ---- filter admission -----------------------------------------------------------

void* qp_filter_new(const int64_t* doc_tokens, int32_t n_docs, const int64_t* stage_tokens,
                    int32_t n_stages, int64_t budget, int64_t arena_pages, int32_t page_tokens,
                    int64_t kept_extra, int64_t limit, const int32_t* order, const int32_t* parent,
                    const int64_t* shared) {
  try {
    return new FilterPlan(doc_tokens, n_docs, stage_tokens, n_stages, budget, arena_pages,
                          page_tokens, kept_extra, limit, order, parent, shared);
  } catch (const Error& e) {
    set_error(e.message.c_str());
  } catch (const std::bad_alloc&) {
    set_error("filter: out of memory");
  }
  return nullptr;
}

void qp_filter_delete(void* plan) { delete static_cast<FilterPlan*>(plan); }

int qp_filter_bind_arena(void* plan, const void* arena, const int64_t* keys, int32_t n) {
  return (int)guarded([&] {
    FilterPlan* f = as<FilterPlan>(plan, "filter");
    if (arena && n != f->borrowing.size()) fail(kValueError, "%d keys for %d documents", n, f->borrowing.size());
    f->borrowing.arena = static_cast<const Arena*>(arena);
    f->borrowing.keys.assign(keys, keys + (keys ? n : 0));
    return (int64_t)kOk;
  });
}

int qp_filter_set_borrow_check(void* plan, int32_t (*check)(int32_t, int32_t, int32_t, void*),
                               void* ctx) {
  return (int)guarded([&] {
    FilterPlan* f = as<FilterPlan>(plan, "filter");
    f->borrowing.check = check;
    f->borrowing.check_ctx = ctx;
    return (int64_t)kOk;
  });
}

int qp_join_set_borrow_check(void* plan, int32_t (*check)(int32_t, int32_t, int32_t, void*),
                             void* ctx) {
  return (int)guarded([&] {
    JoinPlan* j = as<JoinPlan>(plan, "join");
    j->borrowing.check = check;
    j->borrowing.check_ctx = ctx;
    return (int64_t)kOk;
  });
}

static int64_t filter_groups_out(const FilterPlan* f, int32_t* docs, int32_t* stages, uint8_t* fresh,
                                 int64_t cap) {
  const int64_t n = (int64_t)f->groups.size();
  if (docs && n <= cap) {
    for (int64_t i = 0; i < n; ++i) {
      docs[i] = f->groups[i].doc;
      stages[i] = f->groups[i].stage;
      fresh[i] = f->groups[i].fresh;
    }
  }
  return n;
}

int64_t qp_filter_next_chunk(void* plan, int64_t free_pages, int32_t* docs, int32_t* stages,
                             uint8_t* fresh, int64_t cap) {
  return guarded([&] {
    FilterPlan* f = as<FilterPlan>(plan, "filter");
    f->next_chunk(free_pages);
    return filter_groups_out(f, docs, stages, fresh, cap);
  });
}

int qp_filter_stage_chunk(void* plan, void* arena, void* chunk, const void* docs, const void* tails,
                          int64_t preamble, int64_t capacity_extra, int32_t tree_path,
                          int32_t sibling_order, int32_t arena_writes) {
  return (int)guarded([&] {
    FilterPlan* f = as<FilterPlan>(plan, "filter");
    if ((int64_t)f->borrowing.keys.size() != f->borrowing.size())
      fail(kValueError, "filter: arena keys not bound");
    FilterPlan::Prompts p{as<TokenTable>(docs, "docs"), as<TokenTable>(tails, "tails"), preamble,
                          capacity_extra};
    f->stage_chunk(*as<Arena>(arena, "arena"), *as<ChunkBuilder>(chunk, "chunk"), p,
                   tree_path != 0, sibling_order != 0, arena_writes != 0);
    return (int64_t)kOk;
  });
}

int64_t qp_filter_groups(const void* plan, int32_t* docs, int32_t* stages, uint8_t* fresh,
                         int64_t cap) {
  return guarded([&] { return filter_groups_out(as<FilterPlan>(plan, "filter"), docs, stages, fresh, cap); });
}

int qp_filter_report(void* plan, int32_t doc, int32_t stage, int32_t passed, int32_t release,
                     int32_t* free_doc) {
  return (int)guarded([&] {
    *free_doc = as<FilterPlan>(plan, "filter")->report(doc, stage, passed != 0, release != 0);
    return (int64_t)kOk;
  });
}

int64_t qp_filter_report_chunk(void* plan, void* arena, int64_t n, const int32_t* docs,
                               const int32_t* stages, const uint8_t* passed) {
  return guarded([&] {
    FilterPlan* f = as<FilterPlan>(plan, "filter");
    Arena* a = arena ? static_cast<Arena*>(arena) : nullptr;
    int64_t freed = 0;
    for (int64_t i = 0; i < n; ++i) {
      const int32_t d = f->report(docs[i], stages[i], passed[i] != 0, true);
      if (d < 0) continue;
      ++freed;
      if (a) {
        if ((int64_t)f->borrowing.keys.size() <= d) fail(kValueError, "filter: arena keys not bound");
        a->free_key(f->borrowing.keys[d]);
      }
    }
    return freed;
  });
}

int qp_filter_state(const void* plan, int64_t* out) {
  return (int)guarded([&] {
    const FilterPlan* f = as<FilterPlan>(plan, "filter");
    out[0] = f->pending();
    out[1] = f->ready();
    out[2] = f->n_in_flight();
    out[3] = f->survivors;
    out[4] = f->blocked_pages;
    out[5] = f->borrowing.borrowed_tokens;
    out[6] = f->done();
    out[7] = (int64_t)f->groups.size();
    return (int64_t)kOk;
  });
}

int64_t qp_filter_drain_ready(void* plan, int32_t* out, int64_t cap) {
  return guarded([&] {
    std::vector<int32_t> docs = as<FilterPlan>(plan, "filter")->drain_ready();
    if ((int64_t)docs.size() > cap) fail(kValueError, "drain_ready: %zu documents, room for %lld", docs.size(), (long long)cap);
    return copy_out(docs, out, cap);
  });
}

int qp_filter_borrow(const void* plan, int32_t doc, int64_t* out) {
  return (int)guarded([&] {
    const FilterPlan* f = as<FilterPlan>(plan, "filter");
    if (doc < 0 || doc >= f->borrowing.size()) fail(kValueError, "document %d", doc);
    out[0] = f->borrowing.tree_parent(doc);
    out[1] = f->borrowing.tree_shared(doc);
    out[2] = f->borrowing.parent(doc);
    out[3] = f->borrowing.shared(doc);
    out[4] = f->is_resident(doc);
    return (int64_t)kOk;
  });
}

int64_t qp_filter_borrowers(const void* plan, int32_t* out, int64_t cap) {
  return guarded([&] { return copy_out(as<FilterPlan>(plan, "filter")->borrower_counts, out, cap); });
}

// ---- join admission -----------------------------------------------------------------

void* qp_join_new(int32_t n_stages, const int64_t* const* stage_suffix_tokens,
                  const int32_t* stage_sizes, const int64_t* frame_tokens, int64_t budget,
                  int64_t arena_pages, int32_t page_tokens, int32_t temporary_suffix_pages,
                  int64_t canvas_tokens, int32_t n_anchors, const int32_t* tree_parent,
                  const int64_t* tree_shared) {
  try {
    JoinPlan* j = new JoinPlan(n_stages, stage_suffix_tokens, stage_sizes, frame_tokens, budget,
                               arena_pages, page_tokens, temporary_suffix_pages != 0,
                               canvas_tokens);
    try {
      j->set_tree(tree_parent, tree_shared, n_anchors);
    } catch (...) {
      delete j;
      throw;
    }
    return j;
  } catch (const Error& e) {
    set_error(e.message.c_str());
  } catch (const std::bad_alloc&) {
    set_error("join: out of memory");
  }
  return nullptr;
}

void qp_join_delete(void* plan) { delete static_cast<JoinPlan*>(plan); }

int64_t qp_join_register(void* plan, int64_t prefix, int64_t resident_pages,
                         const int32_t* const* lists, const int32_t* list_sizes) {
  return guarded([&] {
    return (int64_t)as<JoinPlan>(plan, "join")->register_anchor(prefix, resident_pages, lists,
                                                                list_sizes);
  });
}

int qp_join_seed(void* plan, const int32_t* order, int32_t n) {
  return (int)guarded([&] {
    as<JoinPlan>(plan, "join")->seed_queue(order, n);
    return (int64_t)kOk;
  });
}

int64_t qp_join_admit(void* plan, int64_t prefix, int64_t resident_pages,
                      const int32_t* const* lists, const int32_t* list_sizes) {
  return guarded([&] {
    return (int64_t)as<JoinPlan>(plan, "join")->admit(prefix, resident_pages, lists, list_sizes);
  });
}

int qp_join_bind_arena(void* plan, const void* arena) {
  return (int)guarded([&] {
    as<JoinPlan>(plan, "join")->borrowing.arena = static_cast<const Arena*>(arena);
    return (int64_t)kOk;
  });
}

int qp_join_set_key(void* plan, int32_t anchor, int64_t key) {
  return (int)guarded([&] {
    JoinPlan* j = as<JoinPlan>(plan, "join");
    if (anchor < 0) fail(kValueError, "anchor %d", anchor);
    auto& keys = j->borrowing.keys;
    if ((int64_t)keys.size() <= anchor) keys.resize(anchor + 1, 0);
    keys[anchor] = key;
    return (int64_t)kOk;
  });
}

int64_t qp_join_next_chunk(void* plan, int64_t free_pages, int32_t* anchor, int32_t* stage,
                           int64_t* start, int64_t* end, uint8_t* carried, int64_t cap) {
  return guarded([&] {
    JoinPlan* j = as<JoinPlan>(plan, "join");
    if (j->borrowing.arena && (int64_t)j->borrowing.keys.size() < j->borrowing.size())
      fail(kValueError, "join: arena keys not bound for every anchor");
    const auto& g = j->next_chunk(free_pages);
    const int64_t n = (int64_t)g.size();
    if (n > cap) fail(kValueError, "join chunk of %lld groups, room for %lld", (long long)n, (long long)cap);
    for (int64_t i = 0; i < n; ++i) {
      anchor[i] = g[i].anchor;
      stage[i] = g[i].stage;
      start[i] = g[i].start;
      end[i] = g[i].end;
      carried[i] = g[i].carried;
    }
    return n;
  });
}

int qp_join_report(void* plan, int32_t anchor, int32_t stage, int64_t start, int64_t end,
                   const uint8_t* bits, int64_t n_bits) {
  return (int)guarded([&] {
    if (n_bits != end - start)
      fail(kStateError, "anchor %d stage %d: %lld answers for partners %lld:%lld", anchor, stage,
           (long long)n_bits, (long long)start, (long long)end);
    as<JoinPlan>(plan, "join")->report(anchor, stage, start, end, bits);
    return (int64_t)kOk;
  });
}

int64_t qp_join_events(void* plan, int32_t settled, int32_t* kinds, int32_t* anchors, int64_t cap) {
  return guarded([&] {
    JoinPlan* j = as<JoinPlan>(plan, "join");
    auto& src = settled ? j->settled : j->events;
    const int64_t n = std::min<int64_t>(cap, (int64_t)src.size());
    for (int64_t i = 0; i < n; ++i) {
      kinds[i] = src[i].first;
      anchors[i] = src[i].second;
    }
    src.erase(src.begin(), src.begin() + n);
    return n;
  });
}

int qp_join_state(const void* plan, int64_t* out) {
  return (int)guarded([&] {
    const JoinPlan* j = as<JoinPlan>(plan, "join");
    out[0] = j->pending_count();
    out[1] = j->ready_count();
    out[2] = j->in_flight;
    out[3] = j->blocked_pages;
    out[4] = j->borrowing.borrowed_tokens;
    out[5] = j->done();
    out[6] = j->n_anchors();
    out[7] = j->buildable_tokens();
    return (int64_t)kOk;
  });
}

int64_t qp_join_partners(const void* plan, int32_t anchor, int32_t stage, int64_t start,
                         int64_t end, int32_t* out) {
  return guarded([&] {
    const JoinPlan* j = as<JoinPlan>(plan, "join");
    if (anchor < 0 || anchor >= j->n_anchors()) fail(kValueError, "anchor %d", anchor);
    if (start < 0 || end < start || end > j->partner_count(anchor, stage))
      fail(kValueError, "anchor %d stage %d: partners %lld:%lld", anchor, stage, (long long)start,
           (long long)end);
    for (int64_t i = start; i < end; ++i) out[i - start] = (int32_t)j->partner_index(anchor, stage, i);
    return end - start;
  });
}

int qp_join_borrow(const void* plan, int32_t anchor, int64_t* out) {
  return (int)guarded([&] {
    const JoinPlan* j = as<JoinPlan>(plan, "join");
    if (anchor < 0 || anchor >= j->borrowing.size()) fail(kValueError, "anchor %d", anchor);
    out[0] = j->borrowing.tree_parent(anchor);
    out[1] = j->borrowing.tree_shared(anchor);
    out[2] = j->borrowing.parent(anchor);
    out[3] = j->borrowing.shared(anchor);
    out[4] = anchor < j->n_anchors() ? j->anchor_stage(anchor) : -1;
    return (int64_t)kOk;
  });
}

int64_t qp_join_borrowers(const void* plan, int32_t* out, int64_t cap) {
  return guarded([&] { return copy_out(as<JoinPlan>(plan, "join")->borrowing.borrowers(), out, cap); });
}

int64_t qp_join_prefix(const void* plan, int32_t anchor) {
  return guarded([&] {
    const JoinPlan* j = as<JoinPlan>(plan, "join");
    if (anchor < 0 || anchor >= j->n_anchors()) fail(kValueError, "anchor %d", anchor);
    return j->prefix[anchor];
  });
}

}  // extern "C"
