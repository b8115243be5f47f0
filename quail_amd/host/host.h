// Internal declarations of libquail_host.so: the host half of the executor
// hot path (page arena, admission, chunk building). Host-only C++17; the C
// ABI over these types is in capi.cpp and include/quail_host.h.
#pragma once

#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

namespace qp {

// Status codes of the C ABI (mirrored in include/quail_host.h).
enum Status : int {
  kOk = 0,
  kNone = 1,       // a request that did not fit: the caller waits or splits
  kKeyError = -1,  // unknown or duplicate key
  kValueError = -2,
  kStateError = -3,  // a broken invariant (the reference raises AssertionError)
  kArenaFull = -4,   // a chunk's temporary pages do not fit the free arena
};

// Thrown inside the library, turned into a status at the C boundary.
struct Error {
  int code;
  std::string message;
};
[[noreturn]] void fail(int code, const char* fmt, ...);

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ----------------------------------------------------------------------------
// Page arena: page accounting plus the borrower holds, deferred frees and
// retention of the KV arena. Keys are integer handles chosen by the caller
// (temporaries get negative handles from the arena itself).
// A retention priority: a tuple of numbers compared lexicographically, as
// Python compares the tuples a retention policy returns (arena.py:170-179;
// cost/retention.py:19-25 returns three: value per page, -next use,
// -document).
struct Priority {
  std::vector<double> v;
};

struct KeyState {
  std::vector<int32_t> pages;  // table order: borrowed pages, then own pages
  int32_t n_borrowed = 0;
  int64_t tokens = 0;
  uint64_t resident_seq = 0;  // allocation order
  bool pinned = false;
  bool retained = false;
  uint64_t retained_version = 0;  // also the retained keys' order
  int64_t retained_tokens = 0;
  int64_t retained_size = 0;  // pages the key alone held when retained
  int64_t queued = 0;         // borrowers queued on the key (a hold)
  uint64_t hold_seq = 0;      // when the hold began
  bool deferred = false;      // freed by its operator while held
};

struct RetainEntry {
  Priority priority;
  uint64_t version;
  int64_t key;
  int64_t pages;
  int64_t tokens;
};

struct EvictEvent {
  int64_t key;
  int64_t tokens;
  int64_t pages;
};

class Arena {
 public:
  Arena(int32_t n_pages, int32_t page_tokens);

  int32_t n_pages() const { return n_pages_; }
  int32_t page_tokens() const { return page_tokens_; }
  int64_t pages_for(int64_t tokens) const { return ceil_div(tokens, page_tokens_); }
  int32_t free_pages() const { return (int32_t)free_.size(); }
  const std::vector<int32_t>& free_stack() const { return free_; }

  bool resident(int64_t key) const { return keys_.count(key) != 0; }
  const KeyState& state(int64_t key) const;
  KeyState& state(int64_t key);

  // --- page accounting ---
  // Own pages for a fresh key behind `borrowed` (a parent's leading pages);
  // false when the free stack is short.
  bool alloc(int64_t key, int64_t tokens, int64_t capacity, const int32_t* borrowed,
             int32_t n_borrowed);
  // The parent's pages for its tokens [start, shared), whole pages.
  std::vector<int32_t> shared_pages(int64_t parent, int64_t shared, int64_t start) const;
  int32_t release_pages(const int32_t* pages, size_t n);
  int32_t free_now(int64_t key);  // ignores holds
  int32_t drop_leading(int64_t key, int64_t pages);
  int32_t rewind(int64_t key, int64_t tokens);  // retention left to the caller
  // Own pages up to capacity; -1 when the free stack is short.
  int64_t grow(int64_t key, int64_t capacity);
  void pin(int64_t key);
  int64_t sole_pages(int64_t key) const;
  void retain(int64_t key, const Priority* priority);
  bool pop_victim(const std::vector<int64_t>& keep, int64_t* key, int64_t* pages,
                  int64_t* tokens);
  void clear_retention_heap() { heap_.clear(); }
  std::vector<int64_t> retained_keys() const;
  std::vector<int64_t> resident_keys() const;
  int64_t retained_pages() const { return retained_pages_; }
  int64_t resident_tokens() const;
  int64_t retained_prefix_tokens() const;
  int64_t retention_cap = -1;  // pages retained KV may keep; -1: no cap yet

  // --- the KV arena's operator-facing rules ---
  // Make a prefix active: grow a resident key, or allocate a fresh one
  // behind its parent's borrowed pages, evicting retained KV as needed.
  // Returns false when the pages do not fit even after eviction.
  bool activate(int64_t key, int64_t tokens, int64_t capacity, int64_t parent,
                int64_t shared);
  int64_t alloc_temporary(int64_t tokens);  // new negative handle, or 0 when short
  void hold(int64_t key, int64_t borrowers);
  void release(int64_t key);
  bool drop_holds(const int64_t* keys, size_t n, bool all);
  int32_t free_key(int64_t key);  // deferred while the key is held
  int32_t evict_key(int64_t key);
  int64_t evict_retained(int64_t pages_needed);  // keys evicted
  void evict_for_pages(int64_t need);
  bool can_borrow(int64_t parent, int64_t shared) const;
  bool held(int64_t key) const;

  std::vector<EvictEvent> events;  // evictions since the caller last drained them
  int64_t evicted_keys = 0, evicted_pages = 0, evicted_prefix_tokens = 0;

 private:
  void forget_retained(KeyState& s);
  std::vector<int64_t> held_keys() const;

  int32_t n_pages_, page_tokens_;
  std::vector<int32_t> free_;   // a stack: back() is the next page handed out
  std::vector<int32_t> holds_;  // keys holding each page
  std::unordered_map<int64_t, KeyState> keys_;
  std::vector<RetainEntry> heap_;  // min-heap on (priority, version)
  int64_t retained_pages_ = 0;
  uint64_t version_ = 0;
  uint64_t resident_seq_ = 0;
  uint64_t hold_seq_ = 0;
  int64_t next_temporary_ = -1;
  int64_t n_held_ = 0;
};

// ----------------------------------------------------------------------------
// Token sources: entries of token ids held as one or more contiguous parts
// of int32 or int64 (numpy arrays, memory-mapped Arrow columns). The library
// only reads them, during a chunk build.
struct TokenPart {
  const void* data;
  int64_t len;
  int32_t elem_bytes;
};

class TokenTable {
 public:
  int64_t add(const TokenPart* parts, int32_t n_parts);
  int64_t length(int64_t entry) const { return lengths_.at(entry); }
  // Append entry[skip:] to out.
  void append(int64_t entry, int64_t skip, std::vector<int64_t>& out) const;
  int64_t size() const { return (int64_t)lengths_.size(); }

 private:
  std::vector<int64_t> first_part_;  // per entry: index into parts_
  std::vector<int32_t> n_parts_;
  std::vector<int64_t> lengths_;
  std::vector<TokenPart> parts_;
};

// The prefix tree of n documents held in one flat buffer of int32 or int64
// ids (document i = ids[offsets[i] .. offsets[i+1])): order[k] is the k-th
// document in sorted order, parent[d] the document d borrows from (-1:
// none), shared[d] the tokens it borrows, a multiple of page_tokens.
void prefix_tree(const void* ids, int32_t elem_bytes, int64_t n, const int64_t* offsets,
                 int64_t page_tokens, int64_t* order, int64_t* parent, int64_t* shared);

// ----------------------------------------------------------------------------
// Admission.

// Which parent each admitted document borrows its KV prefix from.
class Borrowing {
 public:
  static constexpr int32_t kWait = -2;

  void resize(int32_t n);
  int32_t add();  // one more document, no parent
  void set_tree(const int32_t* parent, const int64_t* shared, int32_t n);
  void detach(int32_t doc) { parent_[doc] = -1; shared_[doc] = 0; }
  void skip(int32_t doc) { skipped_[doc] = 1; }
  // -1: pack whole; kWait: the parent is still queued; else the parent.
  int32_t decide(int32_t doc, const std::vector<uint8_t>& in_chunk) const;
  void record(int32_t doc, int32_t parent);
  int32_t size() const { return (int32_t)parent_.size(); }
  int32_t tree_parent(int32_t doc) const { return parent_[doc]; }
  int64_t tree_shared(int32_t doc) const { return shared_[doc]; }
  int32_t parent(int32_t doc) const { return chosen_[doc]; }
  int64_t shared(int32_t doc) const { return chosen_[doc] >= 0 ? shared_[doc] : 0; }
  std::vector<int32_t> borrowers() const;
  int64_t borrowed_tokens = 0;

  // Arena check of a borrow (null: always allowed): whether the parent's
  // pages can serve one, given the documents' arena keys.
  const Arena* arena = nullptr;
  std::vector<int64_t> keys;
  // Or a caller's check (doc, parent, parent in this chunk) -> allowed.
  typedef int32_t (*Check)(int32_t doc, int32_t parent, int32_t same_chunk, void* ctx);
  Check check = nullptr;
  void* check_ctx = nullptr;

 private:
  std::vector<int32_t> parent_;
  std::vector<int64_t> shared_;
  std::vector<uint8_t> admitted_, skipped_;
  std::vector<int32_t> chosen_;
};

struct FilterGroup {
  int32_t doc;
  int32_t stage;
  uint8_t fresh;
};

class FilterPlan {
 public:
  FilterPlan(const int64_t* doc_tokens, int32_t n_docs, const int64_t* stage_tokens,
             int32_t n_stages, int64_t budget, int64_t arena_pages, int32_t page_tokens,
             int64_t kept_extra, int64_t limit, const int32_t* order, const int32_t* parent,
             const int64_t* shared);

  // Groups of the next chunk in admission order; empty when nothing fits.
  const std::vector<FilterGroup>& next_chunk(int64_t free_pages);  // -1: no page budget
  // Record one answer; returns the document to free, or -1.
  int32_t report(int32_t doc, int32_t stage, bool passed, bool release);
  bool done() const;
  std::vector<int32_t> drain_ready();
  int64_t own_tokens(int32_t doc) const { return doc_tokens_[doc] - borrowing.shared(doc); }

  // The chunk of the last next_chunk(), built: the tree path's sibling order,
  // pages activated, one group per admitted entry, parents' holds released.
  struct Prompts {
    const TokenTable* docs;
    const TokenTable* tails;  // one entry per stage
    int64_t preamble;          // shared question preamble tokens
    int64_t capacity_extra;
  };
  void stage_chunk(Arena& arena, class ChunkBuilder& chunk, const Prompts& prompts,
                   bool tree_path, bool sibling_order, bool arena_writes);

  Borrowing borrowing;
  std::vector<int32_t> borrower_counts;
  std::vector<FilterGroup> groups;
  int64_t blocked_pages = 0;
  int64_t survivors = 0;
  int64_t n_in_flight() const { return in_flight_; }
  bool is_resident(int32_t doc) const { return resident_[doc] != 0; }
  int64_t pending() const { return (int64_t)(pending_.size() - head_); }
  int64_t ready() const { return (int64_t)(ready_.size() - ready_head_); }
  const std::vector<int32_t>& tree_rank() const { return rank_; }

 private:
  bool limit_reached() const { return limit_ >= 0 && survivors >= limit_; }
  void push_front(const std::vector<int32_t>& docs);

  std::vector<int64_t> doc_tokens_;
  std::vector<int64_t> stage_tokens_;
  int64_t budget_, page_tokens_, kept_extra_, limit_;
  bool pages_;
  // pending documents: pending_[head_..] in order; front insertion rebuilds
  std::vector<int32_t> pending_;
  size_t head_ = 0;
  std::vector<std::pair<int32_t, int32_t>> ready_;  // (doc, next stage), FIFO
  size_t ready_head_ = 0;
  std::vector<uint8_t> in_flight_flag_, resident_;
  int64_t in_flight_ = 0;
  std::vector<int32_t> rank_;  // position of each document in the tree order
};

// ----------------------------------------------------------------------------
// Chunk building: one forward pass's integer arrays.
struct GroupSpec {
  int64_t key;
  int64_t read_key;  // tree path: the parent whose KV the fresh rows read; 0 = none
  bool has_read;
  bool fresh;        // the prefix is packed (else a kept group: suffixes only)
  int64_t start;     // logical position of the first fresh token
  int64_t f;         // suffix positions start here
  int64_t write_suffix_tokens;
  const TokenTable* prefix_src;
  int64_t prefix_entry;
  int64_t prefix_skip;
  const TokenTable* suffix_src;
  int64_t suffix_begin;  // suffix entries: suffix_idx[suffix_begin .. + n_suffix)
  int32_t n_suffix;
};

enum ArrayId : int {
  kInputIds, kPositions, kFinals, kCuA, kALen, kARead,
  kKvSrc, kKvDst,
  kReadsRows, kReadsCuQ, kReadsUsed, kReadsTable, kReadsSource,
  kUniSrc, kUniDst, kUniUsed, kUniTable, kUniCuQ, kTailSrc, kTailDst, kUniRowDst,
  kNumArrays
};

class ChunkBuilder {
 public:
  void reset();
  void add_group(GroupSpec g, const int32_t* suffix_idx, int32_t n_suffix);
  // Build every array; kArenaFull (as an Error) frees the temporaries made.
  void build(Arena& arena, bool tree_path);

  // results
  struct Array {
    std::vector<int64_t> i64;
    std::vector<int32_t> i32;
    bool wide = true;
    bool present = false;
    int64_t rows = 0, cols = 1;  // 2-D tables: rows x cols
    int64_t bytes() const { return wide ? (int64_t)i64.size() * 8 : (int64_t)i32.size() * 4; }
    const void* data() const { return wide ? (const void*)i64.data() : (const void*)i32.data(); }
  };
  Array arrays[kNumArrays];
  int64_t tokens = 0, max_a = 0;
  bool has_reads = false, has_unified = false;
  int64_t reads_max_q = 0, reads_max_used = 0, reads_rows = 0;
  int64_t uni_max_q = 0, uni_max_used = 0;
  int64_t own_pairs = 0, unified_pairs = 0, unified_kv_rows = 0, read_pairs = 0,
          read_kv_rows = 0;
  std::vector<int64_t> temporaries, fresh_keys;
  std::vector<GroupSpec> groups;
  std::vector<int32_t> suffix_idx;

 private:
  void build_reads(Arena& arena, const std::vector<int64_t>& cu_a);
};

// ----------------------------------------------------------------------------
// Join admission: anchors written into the arena once, partners streamed as
// suffixes that read them, stage by stage.
struct JoinGroup {
  int32_t anchor, stage;
  int64_t start, end;
  uint8_t carried;
};

class JoinPlan {
 public:
  JoinPlan(int32_t n_stages, const int64_t* const* stage_suffix_tokens,
           const int32_t* stage_sizes, const int64_t* frame_tokens, int64_t budget,
           int64_t arena_pages, int32_t page_tokens, bool temporary_suffix_pages,
           int64_t canvas_tokens);

  // Register an anchor (constructor-time or streamed); returns its index.
  // resident_pages < 0: not resident. lists: per stage a partner index list
  // (null for every partner).
  int32_t register_anchor(int64_t prefix, int64_t resident_pages,
                          const int32_t* const* lists, const int32_t* list_sizes);
  void set_tree(const int32_t* parent, const int64_t* shared, int32_t n);
  void seed_queue(const int32_t* order, int32_t n);  // initial pending order
  int32_t admit(int64_t prefix, int64_t resident_pages, const int32_t* const* lists,
                const int32_t* list_sizes);
  const std::vector<JoinGroup>& next_chunk(int64_t free_pages);
  // Record one group's answers; events appended (kind 0 dropped, 1 finished).
  void report(int32_t a, int32_t j, int64_t start, int64_t end, const uint8_t* bits);
  bool done() const;
  int64_t buildable_tokens() const;
  int64_t partner_count(int32_t a, int32_t j) const;
  int64_t partner_index(int32_t a, int32_t j, int64_t i) const;

  Borrowing borrowing;
  std::vector<JoinGroup> groups;
  std::vector<std::pair<int32_t, int32_t>> settled;  // (kind, anchor) not yet taken
  std::vector<std::pair<int32_t, int32_t>> events;   // from report()
  int64_t blocked_pages = 0;
  int64_t in_flight = 0;
  std::vector<int64_t> prefix;  // per anchor prefix tokens
  int32_t n_anchors() const { return (int32_t)anchors_.size(); }
  int64_t pending_count() const { return (int64_t)(pending_.size() - pending_head_); }
  int64_t ready_count() const { return (int64_t)(ready_.size() - ready_head_); }
  int32_t anchor_stage(int32_t a) const { return anchors_[a].stage; }
  int64_t anchor_received(int32_t a, int32_t j) const;

 private:
  struct Anchor {
    int64_t prefix = 0, pages = 0, carried = 0, first = 0;
    int32_t stage = -1;  // -1 queued, >= 0 running, kSettled
    int64_t next = 0;
    std::vector<int32_t> has_list;               // per stage
    std::vector<std::vector<int32_t>> lists;     // per stage partner indices
    std::vector<std::vector<int64_t>> cums;      // per stage cumulative suffix rows
    std::vector<uint8_t> any_true;               // per stage
    std::vector<int64_t> received;               // per stage answers recorded
  };
  static constexpr int32_t kSettled = -2;

  int64_t count(int32_t a, int32_t j) const;
  const std::vector<int64_t>& cum(int32_t a, int32_t j) const;
  int64_t suffix(int32_t a, int32_t j, int64_t i) const;
  int64_t first_cost(int32_t a, int32_t j, int64_t i) const;
  int64_t suffix_page_cost(int32_t a, int32_t j, int64_t i) const;
  const std::vector<int64_t>& page_cum(int32_t a, int32_t j);
  void take(int32_t a, int32_t j, int64_t i, int64_t room, int64_t page_room, int64_t* end,
            int64_t* tokens, int64_t* pages);
  bool launch(int32_t a, int32_t j, int64_t end);

  std::vector<std::vector<int64_t>> stages_;     // per stage suffix rows (+ canvas)
  std::vector<std::vector<int64_t>> stage_cum_;
  std::vector<int64_t> frames_, frame_rows_;
  int64_t budget_, arena_pages_, page_tokens_, extra_ = 0;
  bool temporary_pages_;
  std::vector<Anchor> anchors_;
  std::unordered_map<int64_t, std::vector<int64_t>> page_cum_cache_;
  int64_t page_reserve_ = 0;
  int64_t min_fresh_;
  int64_t zero_cost_ = 0;
  std::vector<int32_t> pending_;  // deque: pending_[pending_head_..]
  size_t pending_head_ = 0;
  std::vector<int32_t> ready_;
  size_t ready_head_ = 0;
  std::vector<int32_t> resident_anchor_;  // anchors registered as resident
};

}  // namespace qp
