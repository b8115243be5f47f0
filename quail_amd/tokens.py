"""Token views and the prefix tree that decides KV page borrowing.

prefix_tree restates quail/execution/tokens.py:514-591 exactly, because the
tree fixes which pages every document reads:
  - documents are visited in ascending order of their token ids' big-endian
    int32 bytes (tokens.py:566), which sorts like the ids themselves with
    shorter prefixes first;
  - a document's shared length is its longest common prefix with the sorted
    predecessor, capped at len - 1 (a document computes its last token) and
    floored to whole pages (tokens.py:580-582);
  - its parent is the predecessor, or the ancestor reached by climbing
    while the ancestor itself borrowed at least that many tokens
    (tokens.py:585-589).
"""

import numpy as np


class PrefixTree:
    """order (parents first), parent per document (or None), shared tokens."""

    def __init__(self, order, parent, shared):
        self.order = order
        self.parent = parent
        self.shared = shared

    @property
    def shared_tokens(self) -> int:
        return sum(self.shared)


def _ids(doc):
    if isinstance(doc, np.ndarray):
        return doc.astype(np.int64, copy=False)
    return np.asarray(list(doc), dtype=np.int64)


def _common(a, b) -> int:
    n = min(a.size, b.size)
    diff = np.flatnonzero(a[:n] != b[:n])
    return int(diff[0]) if diff.size else n


def prefix_tree(documents, page_tokens: int) -> PrefixTree:
    """The prefix tree of a document set (tokens.py:547-591)."""
    n = len(documents)
    arrays = [_ids(documents[i]) for i in range(n)]
    keys = [a.astype(">i4").tobytes() for a in arrays]
    order = sorted(range(n), key=keys.__getitem__)
    parent = [None] * n
    shared = [0] * n
    previous = None
    for index in order:
        if previous is not None:
            lcp = min(_common(arrays[previous], arrays[index]),
                      max(arrays[index].size - 1, 0))
            pages = lcp // page_tokens * page_tokens
            if pages:
                owner = previous
                while parent[owner] is not None and shared[owner] >= pages:
                    owner = parent[owner]
                parent[index] = owner
                shared[index] = pages
        previous = index
    return PrefixTree(order, parent, shared)


def shared_prefix_lengths(sequences) -> list:
    return prefix_tree(sequences, 1).shared


class DocumentPrefixes:
    """Documents with a common token prefix prepended on access (tokens.py:412-429)."""

    def __init__(self, prefix, documents, indices=None):
        self._prefix = np.asarray(prefix, dtype=np.int64)
        self._documents = documents
        self._indices = list(range(len(documents))) if indices is None else list(indices)

    def __len__(self):
        return len(self._indices)

    def __getitem__(self, index):
        if isinstance(index, slice):
            return [self[i] for i in range(*index.indices(len(self)))]
        doc = np.asarray(self._documents[self._indices[index]], dtype=np.int64)
        return np.concatenate([self._prefix, doc])
