// The prefix tree of a document set (quail/execution/tokens.py:547-591): which
// document each document borrows its KV prefix from.
//
// Documents are ordered by their token ids compared as big-endian int32 byte
// strings, i.e. element by element as unsigned 32-bit values with a proper
// prefix first; equal documents keep their input order. Each document shares
// with its predecessor in that order the longest common prefix, capped one
// token short of its own length and floored to whole pages. A document that
// shares a page or more hangs under the nearest document on its
// predecessor's root path whose own share is below that (or the path's
// root), so the path is a stack and each document is pushed and popped once.
#include <algorithm>
#include <numeric>
#include <vector>

#include "host.h"

namespace qp {

namespace {

template <class T>
struct Rows {
  const T* ids;
  const int64_t* offsets;

  const T* begin(int64_t i) const { return ids + offsets[i]; }
  int64_t size(int64_t i) const { return offsets[i + 1] - offsets[i]; }

  // the order of the big-endian int32 bytes of rows a and b
  bool less(int64_t a, int64_t b) const {
    const T* x = begin(a);
    const T* y = begin(b);
    const int64_t n = std::min(size(a), size(b));
    for (int64_t k = 0; k < n; ++k) {
      const uint32_t u = (uint32_t)x[k], v = (uint32_t)y[k];
      if (u != v) return u < v;
    }
    return size(a) < size(b);
  }

  int64_t common(int64_t a, int64_t b) const {
    const T* x = begin(a);
    const T* y = begin(b);
    const int64_t n = std::min(size(a), size(b));
    int64_t k = 0;
    while (k < n && x[k] == y[k]) ++k;
    return k;
  }
};

template <class T>
void build(const Rows<T>& rows, int64_t n, int64_t page_tokens, int64_t* order,
           int64_t* parent, int64_t* shared) {
  std::vector<int64_t> sorted(n);
  std::iota(sorted.begin(), sorted.end(), 0);
  std::stable_sort(sorted.begin(), sorted.end(),
                   [&](int64_t a, int64_t b) { return rows.less(a, b); });
  std::fill(parent, parent + n, -1);
  std::fill(shared, shared + n, 0);
  std::vector<int64_t> path;  // root path of the document visited last
  path.reserve(64);
  for (int64_t k = 0; k < n; ++k) {
    const int64_t doc = sorted[k];
    order[k] = doc;
    int64_t pages = 0;
    if (k > 0) {
      const int64_t keep =
          std::min(rows.common(sorted[k - 1], doc), std::max<int64_t>(rows.size(doc) - 1, 0));
      pages = keep / page_tokens * page_tokens;
    }
    if (pages == 0) {
      path.assign(1, doc);
      continue;
    }
    while (path.size() > 1 && shared[path.back()] >= pages) path.pop_back();
    parent[doc] = path.back();
    shared[doc] = pages;
    path.push_back(doc);
  }
}

}  // namespace

void prefix_tree(const void* ids, int32_t elem_bytes, int64_t n, const int64_t* offsets,
                 int64_t page_tokens, int64_t* order, int64_t* parent, int64_t* shared) {
  if (n < 0) fail(kValueError, "prefix_tree: %lld documents", (long long)n);
  if (page_tokens <= 0) fail(kValueError, "prefix_tree: page_tokens %lld", (long long)page_tokens);
  if (elem_bytes != 4 && elem_bytes != 8)
    fail(kValueError, "prefix_tree: ids of %d bytes (4 or 8)", elem_bytes);
  if (n == 0) return;
  if (!offsets || !order || !parent || !shared)
    fail(kValueError, "prefix_tree: null offsets or output");
  for (int64_t i = 0; i < n; ++i)
    if (offsets[i + 1] < offsets[i])
      fail(kValueError, "prefix_tree: offsets decrease at %lld", (long long)i);
  if (offsets[n] > offsets[0] && !ids) fail(kValueError, "prefix_tree: null ids");
  if (elem_bytes == 4)
    build(Rows<int32_t>{static_cast<const int32_t*>(ids), offsets}, n, page_tokens, order,
          parent, shared);
  else
    build(Rows<int64_t>{static_cast<const int64_t*>(ids), offsets}, n, page_tokens, order,
          parent, shared);
}

}  // namespace qp
