/*
 * quail_host.h - C ABI of libquail_host.so, the host half of the Quail
 * executor hot path: the KV arena's page accounting, filter and join
 * admission, and chunk building (host-only C++, no GPU code).
 *
 * Conventions
 *   - Functions returning int report a status: QP_OK (0), QP_NONE (1, a
 *     request that did not fit: the reference returns None), or a negative
 *     QP_E_* code. Functions returning int64_t return a count or value >= 0,
 *     or a negative QP_E_* code. qp_last_error() holds the message of the
 *     last failure on the calling thread.
 *   - Keys are int64 handles the caller chooses for its arena keys; the
 *     arena hands out negative handles for the temporaries it creates.
 *   - Objects (arena, token table, chunk builder, filter plan, join plan)
 *     are opaque pointers from *_new and released with *_delete. They are
 *     not thread-safe; one host thread drives one executor.
 *   - Token tables hold pointers into caller memory (int32 or int64 ids);
 *     the caller keeps that memory alive while the table is used.
 *
 * Bit-exactness. Page ids, block tables, scatter maps and chunk composition
 * follow the reference's executor (quail/backends/quail/executor/arena.py,
 * pack.py, loop.py) exactly; every function cites the reference code whose
 * results it reproduces.
 */
#ifndef QUAIL_HOST_H
#define QUAIL_HOST_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  QP_OK = 0,
  QP_NONE = 1,            /* did not fit (the reference returns None)        */
  QP_E_KEY = -1,          /* unknown or duplicate key          -> KeyError   */
  QP_E_VALUE = -2,        /* bad argument or geometry          -> ValueError */
  QP_E_STATE = -3,        /* broken invariant                  -> AssertionError */
  QP_E_ARENA_FULL = -4    /* temporaries do not fit            -> ArenaFullError */
};

int qp_version(void);
const char* qp_last_error(void);

/* ------------------------------------------------------------------------
 * Page arena (arena.py:34-276 PageArena, :541-706 KVArena's key rules).
 * A stack of free pages initialised n-1..0 (pages 0, 1, 2, ... first; freed
 * pages reused last-in first-out); per key, the borrowed pages of a parent
 * then its own; per page, the number of keys holding it.
 */
void* qp_arena_new(int32_t n_pages, int32_t page_tokens);
void qp_arena_delete(void* arena);
/* out[16]: n_pages, page_tokens, free_pages, retained_pages, resident_tokens,
 * retained_prefix_tokens, resident keys, evicted_keys, evicted_pages,
 * evicted_prefix_tokens, retention_cap (-1: none), retained keys. */
int qp_arena_stats(const void* arena, int64_t* out);
/* The free stack, bottom to top (the next page handed out is last). */
int64_t qp_arena_free_list(const void* arena, int32_t* out, int64_t cap);
int qp_arena_is_resident(const void* arena, int64_t key);
/* out[8]: tokens, borrowed pages, table pages, pinned, retained,
 * retained tokens, queued borrowers, deferred free. */
int qp_arena_key_info(const void* arena, int64_t key, int64_t* out);
/* A key's block-table pages: borrowed, then own (arena.py:115-117). */
int64_t qp_arena_table(const void* arena, int64_t key, int32_t* out, int64_t cap);
/* PageArena.alloc (arena.py:63-89): QP_NONE when the free stack is short. */
int qp_arena_alloc(void* arena, int64_t key, int64_t tokens, int64_t capacity,
                   const int32_t* borrowed, int32_t n_borrowed);
/* PageArena.shared_pages (arena.py:91-104): pages of tokens [start, shared). */
int64_t qp_arena_shared_pages(const void* arena, int64_t parent, int64_t shared,
                              int64_t start, int32_t* out, int64_t cap);
/* PageArena.release_pages (arena.py:122-130): pages freed. */
int64_t qp_arena_release_pages(void* arena, const int32_t* pages, int64_t n);
/* PageArena.free_key (arena.py:132-139), immediate: pages freed. */
int64_t qp_arena_free_now(void* arena, int64_t key);
/* PageArena.drop_leading: the first pages, borrowed ones first. */
int64_t qp_arena_drop_leading(void* arena, int64_t key, int64_t pages);
/* PageArena.rewind (arena.py:214-229) without its re-retain: pages freed. */
int64_t qp_arena_rewind(void* arena, int64_t key, int64_t tokens);
/* PageArena.grow (arena.py:231-245): *added pages; QP_NONE when short. */
int qp_arena_grow(void* arena, int64_t key, int64_t capacity, int64_t* added);
int qp_arena_pin(void* arena, int64_t key);
/* Pages of the key's table no other key holds. */
int64_t qp_arena_sole_pages(const void* arena, int64_t key);
/* PageArena.retain (arena.py:153-179): a priority tuple of n_priority
 * doubles of any length, compared lexicographically as Python compares
 * tuples, or the default (tokens per sole page) when priority is NULL. */
int qp_arena_retain(void* arena, int64_t key, const double* priority, int32_t n_priority);
/* PageArena.pop_retained_victim (arena.py:192-212): out[3] = key, pages,
 * tokens; QP_NONE when no retained key outside `keep` is left. */
int qp_arena_pop_victim(void* arena, const int64_t* keep, int64_t n_keep, int64_t* out);
int qp_arena_clear_retention(void* arena);
int64_t qp_arena_retained_keys(const void* arena, int64_t* out, int64_t cap);
int64_t qp_arena_resident_keys(const void* arena, int64_t* out, int64_t cap);
int qp_arena_set_retention_cap(void* arena, int64_t cap_pages);
/* KVArena.activate (arena.py:617-658): grow a resident key or allocate a
 * fresh one behind `shared` tokens of `parent` (shared 0: no borrow),
 * evicting retained keys first; QP_NONE when it cannot fit. */
int qp_arena_activate(void* arena, int64_t key, int64_t tokens, int64_t capacity,
                      int64_t parent, int64_t shared);
/* KVArena.alloc_temporary (arena.py:660-664): *key is a new negative
 * handle; QP_NONE when the free stack is short. */
int qp_arena_alloc_temporary(void* arena, int64_t tokens, int64_t* key);
/* KVArena.hold / release / drop_holds (arena.py:668-706): a held key's free
 * is deferred until its last queued borrower is released. drop_holds
 * returns 1 when it dropped any hold. */
int qp_arena_hold(void* arena, int64_t key, int64_t borrowers);
int qp_arena_release(void* arena, int64_t key);
int qp_arena_drop_holds(void* arena, const int64_t* keys, int64_t n, int32_t all);
int qp_arena_held(const void* arena, int64_t key);
/* KVArena.free_key: pages freed now (0 when deferred). */
int64_t qp_arena_free_key(void* arena, int64_t key);
/* KVArena.evict_key / evict_retained (arena.py:560-615): pages freed / keys
 * evicted. Each eviction is logged for qp_arena_drain_evictions. */
int64_t qp_arena_evict_key(void* arena, int64_t key);
int64_t qp_arena_evict_retained(void* arena, int64_t pages_needed);
int64_t qp_arena_drain_evictions(void* arena, int64_t* keys, int64_t* tokens, int64_t* pages,
                                 int64_t cap);

/* ------------------------------------------------------------------------
 * Token tables: entries of token ids as contiguous parts in caller memory.
 */
void* qp_tokens_new(void);
void qp_tokens_delete(void* tokens);
/* One entry of n_parts parts (data[i], lens[i] ids of elem_bytes[i] = 4 or 8
 * bytes); returns its index. */
int64_t qp_tokens_add(void* tokens, const void* const* data, const int64_t* lens,
                      const int32_t* elem_bytes, int32_t n_parts);
/* n entries over one flat buffer of ids: entry i is data[offsets[i] ..
 * offsets[i+1]) (n + 1 offsets, in ids); returns the first entry's index. */
int64_t qp_tokens_add_flat(void* tokens, const void* data, int32_t elem_bytes, int64_t n,
                           const int64_t* offsets);
int64_t qp_tokens_length(const void* tokens, int64_t entry);

/* The prefix tree of n documents (prefix_tree, quail/execution/tokens.py:547-591)
 * over one flat buffer of ids of elem_bytes = 4 or 8 bytes: document i is
 * ids[offsets[i] .. offsets[i+1]) (n + 1 offsets, in ids). Writes order[n]
 * (documents in ascending order of their ids' big-endian int32 bytes, equal
 * documents in input order), parent[n] (the document each borrows from, -1
 * for none) and shared[n] (borrowed tokens: the common prefix with the
 * sorted predecessor, capped one short of the document's length, floored to
 * page_tokens). */
int qp_prefix_tree(const void* ids, int32_t elem_bytes, int64_t n, const int64_t* offsets,
                   int64_t page_tokens, int64_t* order, int64_t* parent, int64_t* shared);

/* ------------------------------------------------------------------------
 * Chunk builder: pack_chunk (loop.py:219-577). Groups are added in chunk
 * order; build() lays out every array of the chunk's Chunk.meta.
 *
 * Array ids (element type): 0 input_ids (i64), 1 positions (i64), 2 finals
 * (i64), 3 cu_a (i32), 4 a_len (i32), 5 a_read (i32), 6 kv_src (i64),
 * 7 kv_dst (i64), 8 reads_rows (i64), 9 reads_cu_q (i32), 10 reads_used
 * (i32), 11 reads_table (i32, rows x cols), 12 reads_source (i32),
 * 13 unified_src (i64), 14 unified_dst (i64), 15 unified_used (i32),
 * 16 unified_table (i32, rows x cols), 17 unified_cu_q (i32), 18 tail_src
 * (i64), 19 tail_dst (i64), 20 unified_row_dst (i64).
 */
#define QP_CHUNK_ARRAYS 21
void* qp_chunk_new(void);
void qp_chunk_delete(void* chunk);
int qp_chunk_reset(void* chunk);
/* One group (a dict of the reference's pack_chunk): its arena key; the read
 * key whose resident KV its fresh rows read (tree path, has_read); fresh:
 * the prefix tokens prefix_src[prefix_entry][prefix_skip:] are packed from
 * logical position `start`; f: the kept length suffix positions start at;
 * write_suffix_tokens: leading rows of the first suffix kept in the key's
 * pages; suffixes: suffix_src entries. */
int qp_chunk_add_group(void* chunk, int64_t key, int64_t read_key, int32_t has_read,
                       int32_t fresh, int64_t start, int64_t f, int64_t write_suffix_tokens,
                       const void* prefix_src, int64_t prefix_entry, int64_t prefix_skip,
                       const void* suffix_src, const int32_t* suffix_entries,
                       int32_t n_suffix);
/* Build over the arena's current pages. QP_E_ARENA_FULL when a unified
 * suffix's temporary pages do not fit (the temporaries made are freed). */
int qp_chunk_build(void* chunk, void* arena, int32_t tree_path);
/* out[16]: tokens, max_a, has_reads, reads_max_q, reads_max_used,
 * reads_rows, has_unified, unified_max_q, unified_max_used, own_pairs,
 * unified_pairs, unified_kv_rows, read_pairs, read_kv_rows, temporaries,
 * fresh keys. */
int qp_chunk_summary(const void* chunk, int64_t* out);
/* Per array id: out[4 * id ..] = present, elements, rows, cols. */
int qp_chunk_arrays(const void* chunk, int64_t* out);
/* Copy every present array into dst (16-byte aligned slots, in id order);
 * offsets[id] = byte offset or -1. Returns the bytes used, or QP_E_VALUE
 * when cap is short (qp_chunk_emit(chunk, NULL, 0, offsets) sizes it). */
int64_t qp_chunk_emit(const void* chunk, void* dst, int64_t cap, int64_t* offsets);
int64_t qp_chunk_temporaries(const void* chunk, int64_t* out, int64_t cap);
int64_t qp_chunk_fresh_keys(const void* chunk, int64_t* out, int64_t cap);

/* ------------------------------------------------------------------------
 * Filter admission (pack.py:131-209 Borrowing, :647-836 FilterAdmission).
 * arena_pages < 0: no page accounting; limit < 0: none; order / parent /
 * shared: the prefix tree (NULL: none).
 */
void* qp_filter_new(const int64_t* doc_tokens, int32_t n_docs, const int64_t* stage_tokens,
                    int32_t n_stages, int64_t budget, int64_t arena_pages, int32_t page_tokens,
                    int64_t kept_extra, int64_t limit, const int32_t* order,
                    const int32_t* parent, const int64_t* shared);
void qp_filter_delete(void* plan);
/* Borrow checks against the arena (loop.py:1168-1182); keys[doc] is each
 * document's arena key. arena NULL: every borrow allowed. */
int qp_filter_bind_arena(void* plan, const void* arena, const int64_t* keys, int32_t n);
/* A caller's borrow check instead (Borrowing.can_borrow, pack.py:184-194):
 * check(doc, parent, parent admitted in this chunk, ctx) != 0 allows it. */
int qp_filter_set_borrow_check(void* plan, int32_t (*check)(int32_t, int32_t, int32_t, void*),
                               void* ctx);
int qp_join_set_borrow_check(void* plan, int32_t (*check)(int32_t, int32_t, int32_t, void*),
                             void* ctx);
/* FilterAdmission.next_chunk (pack.py:723-780): groups (doc, stage, fresh);
 * free_pages < 0: no page budget. Returns the group count. */
int64_t qp_filter_next_chunk(void* plan, int64_t free_pages, int32_t* docs, int32_t* stages,
                             uint8_t* fresh, int64_t cap);
/* The filter loop's chunk step (loop.py:1482-1505): on the tree path the
 * groups are put in sibling order, fresh documents' pages are activated
 * (holding their borrowers' parents), every group's spec is added to the
 * chunk (loop.py:1344-1359) and the chunk is built; then each fresh
 * document's tree parent is released. docs / tails are token tables (one
 * entry per document / per stage). */
int qp_filter_stage_chunk(void* plan, void* arena, void* chunk, const void* docs,
                          const void* tails, int64_t preamble, int64_t capacity_extra,
                          int32_t tree_path, int32_t sibling_order, int32_t arena_writes);
/* The groups of the last chunk, in chunk order. */
int64_t qp_filter_groups(const void* plan, int32_t* docs, int32_t* stages, uint8_t* fresh,
                         int64_t cap);
/* FilterAdmission.report (pack.py:784-805): *free_doc = the document whose
 * pages the caller frees, or -1. */
int qp_filter_report(void* plan, int32_t doc, int32_t stage, int32_t passed, int32_t release,
                     int32_t* free_doc);
/* A chunk's answers at once, in chunk order: qp_filter_report with release
 * for each (doc, stage, passed), freeing each returned document's key in
 * the arena (KVArena.free_key) before the next report, as the reference's
 * loop does (loop.py:1396-1423). Returns the documents freed. */
int64_t qp_filter_report_chunk(void* plan, void* arena, int64_t n, const int32_t* docs,
                               const int32_t* stages, const uint8_t* passed);
/* out[8]: pending, ready, in flight, survivors, blocked_pages,
 * borrowed_tokens, done, groups of the last chunk. */
int qp_filter_state(const void* plan, int64_t* out);
int64_t qp_filter_drain_ready(void* plan, int32_t* out, int64_t cap);
/* out[5]: tree parent (-1), tree shared, chosen parent (-1), chosen shared,
 * resident in the plan. */
int qp_filter_borrow(const void* plan, int32_t doc, int64_t* out);
int64_t qp_filter_borrowers(const void* plan, int32_t* out, int64_t cap);

/* ------------------------------------------------------------------------
 * Join admission (pack.py:212-644 JoinAdmission).
 */
void* qp_join_new(int32_t n_stages, const int64_t* const* stage_suffix_tokens,
                  const int32_t* stage_sizes, const int64_t* frame_tokens, int64_t budget,
                  int64_t arena_pages, int32_t page_tokens, int32_t temporary_suffix_pages,
                  int64_t canvas_tokens, int32_t n_anchors, const int32_t* tree_parent,
                  const int64_t* tree_shared);
void qp_join_delete(void* plan);
/* Anchor registration, in index order, for the n_anchors of qp_join_new;
 * resident_pages < 0: not resident; lists[j] NULL: every stage-j partner. */
int64_t qp_join_register(void* plan, int64_t prefix, int64_t resident_pages,
                         const int32_t* const* lists, const int32_t* list_sizes);
/* The initial queue: resident anchors, then `order` (NULL: index order). */
int qp_join_seed(void* plan, const int32_t* order, int32_t n);
/* JoinAdmission.admit (pack.py:423-435): a streamed anchor; its index. */
int64_t qp_join_admit(void* plan, int64_t prefix, int64_t resident_pages,
                      const int32_t* const* lists, const int32_t* list_sizes);
int qp_join_bind_arena(void* plan, const void* arena);
int qp_join_set_key(void* plan, int32_t anchor, int64_t key);
/* JoinAdmission.next_chunk (pack.py:500-583): groups (anchor, stage, start,
 * end, carried). */
int64_t qp_join_next_chunk(void* plan, int64_t free_pages, int32_t* anchor, int32_t* stage,
                           int64_t* start, int64_t* end, uint8_t* carried, int64_t cap);
/* JoinAdmission.report (pack.py:587-638): n_bits = end - start answers. */
int qp_join_report(void* plan, int32_t anchor, int32_t stage, int64_t start, int64_t end,
                   const uint8_t* bits, int64_t n_bits);
/* Drain events: from report() (settled = 0) or anchors settled without a
 * chunk (settled = 1). kinds: 0 dropped, 1 finished. */
int64_t qp_join_events(void* plan, int32_t settled, int32_t* kinds, int32_t* anchors,
                       int64_t cap);
/* out[8]: pending, ready, in flight, blocked_pages, borrowed_tokens, done,
 * anchors, buildable tokens. */
int qp_join_state(const void* plan, int64_t* out);
/* Stage partner indices of anchor's group [start, end). */
int64_t qp_join_partners(const void* plan, int32_t anchor, int32_t stage, int64_t start,
                         int64_t end, int32_t* out);
int qp_join_borrow(const void* plan, int32_t anchor, int64_t* out);
int64_t qp_join_borrowers(const void* plan, int32_t* out, int64_t cap);
int64_t qp_join_prefix(const void* plan, int32_t anchor);

#ifdef __cplusplus
}
#endif

#endif /* QUAIL_HOST_H */
