// Page arena: the free-page stack, per-key page lists with borrowed prefixes,
// page refcounts, borrower holds with deferred frees, and retained-KV
// eviction by priority.
//
// Rules fixed by the reference, since page ids reach the kernels through
// block tables and must match bit for bit
// (quail/backends/quail/executor/arena.py:34-276, :541-706):
//   - a fresh arena hands out pages 0, 1, 2, ...; freed pages are reused
//     last-in first-out (the free list is a stack initialised n-1 .. 0);
//   - a key's table is its borrowed pages (a parent's leading pages), then
//     its own; pages are released in that order;
//   - a page returns to the stack when the last key holding it lets go;
//   - retained keys are evicted lowest priority first (default priority:
//     retained tokens per page the key alone holds), ties by retain order.
#include <algorithm>
#include <cstdarg>
#include <cstdio>

#include "host.h"

namespace qp {

void fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  throw Error{code, buf};
}

namespace {

// Heap order: smaller priority first (lexicographic, a shorter tuple before
// a longer one it prefixes), then older retain first.
bool entry_after(const RetainEntry& a, const RetainEntry& b) {
  const std::vector<double>& x = a.priority.v;
  const std::vector<double>& y = b.priority.v;
  const size_t n = std::min(x.size(), y.size());
  for (size_t i = 0; i < n; ++i) {
    if (x[i] != y[i]) return x[i] > y[i];
  }
  if (x.size() != y.size()) return x.size() > y.size();
  return a.version > b.version;
}

}  // namespace

Arena::Arena(int32_t n_pages, int32_t page_tokens) : n_pages_(n_pages), page_tokens_(page_tokens) {
  if (n_pages < 0 || page_tokens <= 0) fail(kValueError, "arena of %d pages x %d tokens", n_pages, page_tokens);
  free_.resize(n_pages);
  for (int32_t i = 0; i < n_pages; ++i) free_[i] = n_pages - 1 - i;
  holds_.assign(n_pages, 0);
}

const KeyState& Arena::state(int64_t key) const {
  auto it = keys_.find(key);
  if (it == keys_.end()) fail(kKeyError, "key %lld is not resident", (long long)key);
  return it->second;
}

KeyState& Arena::state(int64_t key) {
  auto it = keys_.find(key);
  if (it == keys_.end()) fail(kKeyError, "key %lld is not resident", (long long)key);
  return it->second;
}

bool Arena::alloc(int64_t key, int64_t tokens, int64_t capacity, const int32_t* borrowed,
                  int32_t n_borrowed) {
  if (keys_.count(key)) fail(kKeyError, "key %lld already resident", (long long)key);
  if (capacity < tokens) fail(kValueError, "capacity_tokens must cover logical tokens");
  if ((int64_t)n_borrowed * page_tokens_ > tokens)
    fail(kValueError, "a key cannot borrow past its own tokens");
  const int64_t need = pages_for(capacity) - n_borrowed;
  if (need > (int64_t)free_.size()) return false;
  KeyState s;
  s.pages.reserve(n_borrowed + std::max<int64_t>(need, 0));
  s.pages.assign(borrowed, borrowed + n_borrowed);
  for (int64_t i = 0; i < need; ++i) {
    s.pages.push_back(free_.back());
    free_.pop_back();
  }
  for (int32_t p : s.pages) holds_[p] += 1;
  s.n_borrowed = n_borrowed;
  s.tokens = tokens;
  s.resident_seq = ++resident_seq_;
  keys_.emplace(key, std::move(s));
  return true;
}

std::vector<int32_t> Arena::shared_pages(int64_t parent, int64_t shared, int64_t start) const {
  if ((shared - start) % page_tokens_ || start % page_tokens_)
    fail(kValueError, "a borrowed prefix is a whole number of pages");
  auto it = keys_.find(parent);
  if (it == keys_.end()) fail(kKeyError, "borrow parent %lld is not resident", (long long)parent);
  if (shared > it->second.tokens) fail(kValueError, "the parent holds fewer tokens than borrowed");
  const auto& pages = it->second.pages;
  const int64_t lo = std::min<int64_t>(start / page_tokens_, pages.size());
  const int64_t hi = std::min<int64_t>(shared / page_tokens_, pages.size());
  return std::vector<int32_t>(pages.begin() + lo, pages.begin() + std::max(lo, hi));
}

int32_t Arena::release_pages(const int32_t* pages, size_t n) {
  int32_t freed = 0;
  for (size_t i = 0; i < n; ++i) {
    const int32_t p = pages[i];
    if (--holds_[p] == 0) {
      free_.push_back(p);
      ++freed;
    }
  }
  return freed;
}

void Arena::forget_retained(KeyState& s) {
  if (s.retained) {
    retained_pages_ -= s.retained_size;
    s.retained = false;
    s.retained_size = 0;
  }
}

int32_t Arena::free_now(int64_t key) {
  auto it = keys_.find(key);
  if (it == keys_.end()) fail(kKeyError, "key %lld is not resident", (long long)key);
  KeyState s = std::move(it->second);
  forget_retained(s);
  if (s.queued > 0) --n_held_;
  keys_.erase(it);
  return release_pages(s.pages.data(), s.pages.size());
}

int32_t Arena::drop_leading(int64_t key, int64_t pages) {
  KeyState& s = state(key);
  pages = std::min<int64_t>(pages, s.pages.size());
  std::vector<int32_t> dropped(s.pages.begin(), s.pages.begin() + pages);
  s.pages.erase(s.pages.begin(), s.pages.begin() + pages);
  s.n_borrowed = (int32_t)std::max<int64_t>(0, s.n_borrowed - pages);
  return release_pages(dropped.data(), dropped.size());
}

int32_t Arena::rewind(int64_t key, int64_t tokens) {
  KeyState& s = state(key);
  const int64_t borrowed_tokens = (int64_t)s.n_borrowed * page_tokens_;
  const int64_t capacity = (int64_t)s.pages.size() * page_tokens_;
  if (tokens < borrowed_tokens || tokens > capacity)
    fail(kValueError, "rewind tokens leave the resident capacity");
  const int64_t keep = pages_for(tokens);
  std::vector<int32_t> released(s.pages.begin() + keep, s.pages.end());
  s.pages.resize(keep);
  s.tokens = tokens;
  return release_pages(released.data(), released.size());
}

int64_t Arena::grow(int64_t key, int64_t capacity) {
  KeyState& s = state(key);
  const int64_t need = pages_for(capacity) - (int64_t)s.pages.size();
  if (need <= 0) return 0;
  if (need > (int64_t)free_.size()) return -1;
  for (int64_t i = 0; i < need; ++i) {
    const int32_t p = free_.back();
    free_.pop_back();
    holds_[p] += 1;
    s.pages.push_back(p);
  }
  return need;
}

void Arena::pin(int64_t key) {
  KeyState& s = state(key);
  forget_retained(s);
  s.pinned = true;
}

int64_t Arena::sole_pages(int64_t key) const {
  const KeyState& s = state(key);
  int64_t n = 0;
  for (int32_t p : s.pages) n += holds_[p] == 1;
  return n;
}

void Arena::retain(int64_t key, const Priority* priority) {
  KeyState& s = state(key);
  s.pinned = false;
  forget_retained(s);
  const int64_t pages = sole_pages(key);
  s.retained = true;
  s.retained_tokens = s.tokens;
  s.retained_size = pages;
  retained_pages_ += pages;
  s.retained_version = ++version_;
  RetainEntry e;
  if (priority) {
    e.priority = *priority;
  } else {
    e.priority.v.assign(1, (double)s.tokens / (double)std::max<int64_t>(1, pages));
  }
  e.version = s.retained_version;
  e.key = key;
  e.pages = pages;
  e.tokens = s.tokens;
  heap_.push_back(e);
  std::push_heap(heap_.begin(), heap_.end(), entry_after);
}

bool Arena::pop_victim(const std::vector<int64_t>& keep, int64_t* key, int64_t* pages,
                       int64_t* tokens) {
  std::vector<RetainEntry> passed;
  bool found = false;
  while (!heap_.empty()) {
    std::pop_heap(heap_.begin(), heap_.end(), entry_after);
    RetainEntry e = heap_.back();
    heap_.pop_back();
    auto it = keys_.find(e.key);
    if (it == keys_.end() || !it->second.retained || it->second.retained_version != e.version)
      continue;  // stale: re-retained, pinned or freed since
    if (std::find(keep.begin(), keep.end(), e.key) != keep.end()) {
      passed.push_back(e);
      continue;
    }
    forget_retained(it->second);
    *key = e.key;
    *pages = e.pages;
    *tokens = e.tokens;
    found = true;
    break;
  }
  for (const RetainEntry& e : passed) {
    heap_.push_back(e);
    std::push_heap(heap_.begin(), heap_.end(), entry_after);
  }
  return found;
}

std::vector<int64_t> Arena::retained_keys() const {
  std::vector<std::pair<uint64_t, int64_t>> order;
  for (const auto& kv : keys_)
    if (kv.second.retained) order.emplace_back(kv.second.retained_version, kv.first);
  std::sort(order.begin(), order.end());
  std::vector<int64_t> out;
  for (const auto& o : order) out.push_back(o.second);
  return out;
}

std::vector<int64_t> Arena::resident_keys() const {
  std::vector<std::pair<uint64_t, int64_t>> order;
  for (const auto& kv : keys_) order.emplace_back(kv.second.resident_seq, kv.first);
  std::sort(order.begin(), order.end());
  std::vector<int64_t> out;
  for (const auto& o : order) out.push_back(o.second);
  return out;
}

int64_t Arena::resident_tokens() const {
  int64_t n = 0;
  for (const auto& kv : keys_) n += kv.second.tokens;
  return n;
}

int64_t Arena::retained_prefix_tokens() const {
  int64_t n = 0;
  for (const auto& kv : keys_)
    if (kv.second.retained) n += kv.second.tokens;
  return n;
}

// ---- the KV arena's rules over the accounting ----------------------------

bool Arena::held(int64_t key) const {
  auto it = keys_.find(key);
  return it != keys_.end() && it->second.queued > 0;
}

std::vector<int64_t> Arena::held_keys() const {
  std::vector<int64_t> out;
  if (n_held_ == 0) return out;
  for (const auto& kv : keys_)
    if (kv.second.queued > 0) out.push_back(kv.first);
  return out;
}

bool Arena::can_borrow(int64_t parent, int64_t shared) const {
  auto it = keys_.find(parent);
  return it != keys_.end() && shared <= it->second.tokens;
}

int32_t Arena::evict_key(int64_t key) {
  const int64_t tokens = state(key).tokens;
  const int32_t pages = free_key(key);
  evicted_keys += 1;
  evicted_pages += pages;
  evicted_prefix_tokens += tokens;
  events.push_back(EvictEvent{key, tokens, pages});
  return pages;
}

int64_t Arena::evict_retained(int64_t pages_needed) {
  const int64_t start = free_pages();
  int64_t n = 0;
  while (free_pages() - start < pages_needed) {
    int64_t key, pages, tokens;
    if (!pop_victim(held_keys(), &key, &pages, &tokens)) break;
    evict_key(key);
    ++n;
  }
  return n;
}

void Arena::evict_for_pages(int64_t need) {
  while (free_pages() < need) {
    int64_t key, pages, tokens;
    if (!pop_victim(held_keys(), &key, &pages, &tokens)) break;
    evict_key(key);
  }
}

bool Arena::activate(int64_t key, int64_t tokens, int64_t capacity, int64_t parent,
                     int64_t shared) {
  auto it = keys_.find(key);
  if (it != keys_.end()) {
    pin(key);
    const int64_t need = std::max<int64_t>(0, pages_for(capacity) - (int64_t)it->second.pages.size());
    evict_for_pages(need);
    if (need > free_pages()) return false;
    grow(key, capacity);
    keys_.at(key).tokens = tokens;
    return true;
  }
  std::vector<int32_t> borrowed;
  if (shared > 0) borrowed = shared_pages(parent, shared, 0);
  evict_for_pages(pages_for(capacity) - (int64_t)borrowed.size());
  // the borrow is planned again after eviction, which may have taken the parent
  if (shared > 0) borrowed = shared_pages(parent, shared, 0);
  if (!alloc(key, tokens, capacity, borrowed.data(), (int32_t)borrowed.size())) return false;
  pin(key);
  return true;
}

int64_t Arena::alloc_temporary(int64_t tokens) {
  const int64_t key = next_temporary_;
  if (!alloc(key, tokens, tokens, nullptr, 0)) return 0;
  --next_temporary_;
  return key;
}

void Arena::hold(int64_t key, int64_t borrowers) {
  if (borrowers <= 0) return;
  KeyState& s = state(key);
  if (s.queued == 0) {
    s.hold_seq = ++hold_seq_;
    ++n_held_;
  }
  s.queued += borrowers;
}

void Arena::release(int64_t key) {
  auto it = keys_.find(key);
  if (it == keys_.end() || it->second.queued == 0) return;
  if (--it->second.queued == 0) {
    --n_held_;
    if (it->second.deferred) {
      it->second.deferred = false;
      free_key(key);
    }
  }
}

bool Arena::drop_holds(const int64_t* keys, size_t n, bool all) {
  std::vector<int64_t> order;
  if (all) {
    std::vector<std::pair<uint64_t, int64_t>> seq;
    for (const auto& kv : keys_)
      if (kv.second.queued > 0) seq.emplace_back(kv.second.hold_seq, kv.first);
    std::sort(seq.begin(), seq.end());
    for (const auto& s : seq) order.push_back(s.second);
  } else {
    for (size_t i = 0; i < n; ++i)
      if (held(keys[i]) && std::find(order.begin(), order.end(), keys[i]) == order.end())
        order.push_back(keys[i]);
  }
  for (int64_t key : order) {
    KeyState& s = keys_.at(key);
    s.queued = 0;
    --n_held_;
    if (s.deferred) {
      s.deferred = false;
      free_key(key);
    }
  }
  return !order.empty();
}

int32_t Arena::free_key(int64_t key) {
  KeyState& s = state(key);
  if (s.queued > 0) {
    s.deferred = true;
    return 0;
  }
  return free_now(key);
}

}  // namespace qp
