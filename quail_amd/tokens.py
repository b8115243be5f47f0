"""Token views, the on-disk token store, and the prefix tree that decides
KV page borrowing.

Token store files are Arrow IPC files, memory mapped, in the reference's
layout (quail/execution/tokens.py:193-210, :316-319): one record batch per
source batch with a `__quail_token_ids` large_list<int> column and a
`__quail_token_count` int64 column, schema metadata quail.kind=token_store;
a column store holds one copied source column (quail.kind=column_store). A
document read from a store is a TokenView over the mapped buffer; slicing
and prefixing build views and chains, and the packer copies the ids once,
into its pinned staging buffer.

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

import bisect
import contextlib
import os

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


def _integer_ids(seq):
    """A sequence's ids as a 1-D integer array; TypeError if they are not
    integers (a test tokenizer's words)."""
    a = token_array(seq)
    if a.size == 0:
        return np.empty(0, dtype=np.int32)
    if a.dtype.kind not in "iu":
        raise TypeError(f"token ids of dtype {a.dtype}")
    return a.reshape(-1)


def flat_tokens(documents, prefix=None):
    """Every document's ids in one buffer: (ids, offsets) with document i at
    ids[offsets[i]:offsets[i+1]], each preceded by `prefix` if given. The ids
    are int32 when every source part is, else int64. A source with its own
    flat_tokens() (RowPrompts, TokenStore) hands over its buffer; otherwise
    each document is read once. TypeError for ids that are not integers."""
    p = None if prefix is None else _integer_ids(np.asarray(prefix))
    if hasattr(documents, "flat_tokens"):
        ids, offsets = documents.flat_tokens()
        return (ids, offsets) if p is None else _prefixed(p, ids, offsets)
    arrays = [_integer_ids(documents[i]) for i in range(len(documents))]
    lengths = np.fromiter((a.size for a in arrays), dtype=np.int64, count=len(arrays))
    offsets = np.zeros(len(arrays) + 1, dtype=np.int64)
    np.cumsum(lengths + (0 if p is None else p.size), out=offsets[1:])
    narrow = all(a.dtype == np.int32 for a in arrays) and (p is None or _fits_int32(p))
    dtype = np.int32 if narrow else np.int64
    if p is not None:
        p = p.astype(dtype, copy=False)
        arrays = [x for a in arrays for x in (p, a)]
    ids = np.concatenate(arrays).astype(dtype, copy=False) if arrays else \
        np.empty(0, dtype=dtype)
    return ids, offsets


def _fits_int32(a):
    return a.dtype == np.int32 or not a.size or (
        int(a.min()) >= -2**31 and int(a.max()) < 2**31)


def _prefixed(prefix, ids, offsets):
    """(ids, offsets) of documents given as (ids, offsets), each preceded by
    the integer array prefix, built with array operations (no per-document
    work)."""
    n = offsets.size - 1
    lengths = np.diff(offsets)
    p = prefix.size
    out_offsets = np.zeros(n + 1, dtype=np.int64)
    np.cumsum(lengths + p, out=out_offsets[1:])
    narrow = ids.dtype == np.int32 and _fits_int32(prefix)
    out = np.empty(int(out_offsets[-1]), dtype=np.int32 if narrow else np.int64)
    is_doc = np.ones(out.size, dtype=bool)
    if p and n:
        at = (out_offsets[:-1, None] + np.arange(p, dtype=np.int64)).reshape(-1)
        is_doc[at] = False
        out[at] = np.tile(prefix.astype(out.dtype, copy=False), n)
    out[is_doc] = ids[int(offsets[0]):int(offsets[-1])] if n else ids[:0]
    return out, out_offsets


def _prefix_tree_items(documents, page_tokens):
    """prefix_tree for tokens that are not integers (tokens.py:560-564):
    sorted as tuples, the common prefix counted item by item."""
    n = len(documents)
    items = [tuple(documents[i]) for i in range(n)]

    def common(a, b):
        k = 0
        while k < min(len(a), len(b)) and a[k] == b[k]:
            k += 1
        return k

    order = sorted(range(n), key=items.__getitem__)
    parent, shared, path = [None] * n, [0] * n, []
    for prev, doc in zip([None] + order[:-1], order):
        pages = 0
        if prev is not None:
            keep = min(common(items[prev], items[doc]), max(len(items[doc]) - 1, 0))
            pages = keep // page_tokens * page_tokens
        if not pages:
            path = [doc]
            continue
        while len(path) > 1 and shared[path[-1]] >= pages:
            path.pop()
        parent[doc] = path[-1]
        shared[doc] = pages
        path.append(doc)
    return PrefixTree(order, parent, shared)


def prefix_tree(documents, page_tokens: int) -> PrefixTree:
    """The prefix tree of a document set (tokens.py:547-591), built by the
    host library (qp_prefix_tree) over the documents' ids in one buffer.

    Documents are visited in the order of their token ids as big-endian
    int32 bytes. Each one shares with its predecessor in that order the
    longest common prefix, capped one token short of its own length and
    rounded down to whole pages; a document that shares a page or more hangs
    under the nearest document on its predecessor's root path whose own
    shared length is below that (or the path's root)."""
    if page_tokens <= 0:
        raise ValueError(f"page_tokens must be positive, got {page_tokens}")
    try:
        ids, offsets = flat_tokens(documents)
    except (TypeError, ValueError):
        return _prefix_tree_items(documents, page_tokens)
    from . import _host
    n = offsets.size - 1
    ids = np.ascontiguousarray(ids)
    offsets = np.ascontiguousarray(offsets, dtype=np.int64)
    order = np.empty(n, dtype=np.int64)
    parent = np.empty(n, dtype=np.int64)
    shared = np.empty(n, dtype=np.int64)
    _host.call("qp_prefix_tree", ids.ctypes.data, ids.itemsize, n, offsets.ctypes.data,
               page_tokens, order.ctypes.data, parent.ctypes.data, shared.ctypes.data)
    return PrefixTree(order.tolist(), [None if p < 0 else p for p in parent.tolist()],
                      shared.tolist())


def shared_prefix_lengths(sequences) -> list:
    return prefix_tree(sequences, 1).shared


class _Rows:
    """A read-only sequence whose item i comes from self.row(i): slices give
    lists, negative indices count from the end, anything else out of range
    raises IndexError."""

    def __getitem__(self, index):
        n = len(self)
        if isinstance(index, slice):
            return [self.row(i) for i in range(*index.indices(n))]
        i = int(index)
        if i < 0:
            i += n
        if not 0 <= i < n:
            raise IndexError(index)
        return self.row(i)

    def __iter__(self):
        return (self.row(i) for i in range(len(self)))


class DocumentPrefixes(_Rows):
    """Documents with a common token prefix prepended on access (tokens.py:412-429)."""

    def __init__(self, prefix, documents, indices=None):
        self.prefix = np.asarray(prefix, dtype=np.int64)
        self.documents = documents
        self.picked = np.arange(len(documents)) if indices is None else np.asarray(indices)

    def __len__(self):
        return len(self.picked)

    def row(self, i):
        doc = np.asarray(self.documents[int(self.picked[i])], dtype=np.int64)
        return np.concatenate([self.prefix, doc])


# ----------------------------------------------------------------- token views

class TokenView:
    """One contiguous run of token ids backed by an Arrow array (tokens.py:13-42).

    Integer indexing returns a Python int, a unit-step slice another view
    over the same buffer, numpy() the ids without a copy.
    """

    def __init__(self, values):
        self._values = values

    def __len__(self):
        return len(self._values)

    def __getitem__(self, index):
        if isinstance(index, slice):
            start, stop, step = index.indices(len(self))
            if step != 1:
                return self.numpy()[index].tolist()
            return TokenView(self._values.slice(start, max(stop - start, 0)))
        return self._values[index].as_py()

    def __iter__(self):
        return iter(self.numpy().tolist())

    def numpy(self):
        return self._values.to_numpy(zero_copy_only=True)

    def __array__(self, dtype=None, copy=None):
        a = self.numpy()
        return a if dtype is None else a.astype(dtype, copy=False)

    @property
    def arrow_array(self):
        return self._values

    @property
    def token_parts(self):
        return (self,)


class TokenChain:
    """Token parts read in order without copying them (tokens.py:45-100).

    Nested chains flatten and empty parts drop out; a unit-step slice is a
    chain of the sliced parts.
    """

    def __init__(self, *parts):
        flat = []
        for part in parts:
            if isinstance(part, TokenChain):
                flat.extend(part.token_parts)
            elif len(part):
                flat.append(part)
        self._parts = tuple(flat)
        self._ends = np.cumsum([len(p) for p in self._parts], dtype=np.int64)

    def __len__(self):
        return int(self._ends[-1]) if len(self._parts) else 0

    def __iter__(self):
        for part in self._parts:
            yield from part

    def __getitem__(self, index):
        n = len(self)
        if isinstance(index, slice):
            start, stop, step = index.indices(n)
            if step != 1:
                return token_array(self)[index].tolist()
            out, begin = [], 0
            for part, end in zip(self._parts, self._ends.tolist()):
                if end > start and begin < stop:
                    out.append(part[max(0, start - begin):min(stop, end) - begin])
                begin = end
                if begin >= stop:
                    break
            return TokenChain(*out)
        if index < 0:
            index += n
        if not 0 <= index < n:
            raise IndexError(index)
        which = int(np.searchsorted(self._ends, index, side="right"))
        begin = int(self._ends[which - 1]) if which else 0
        return self._parts[which][index - begin]

    def __array__(self, dtype=None, copy=None):
        a = token_array(self)
        return a if dtype is None else a.astype(dtype, copy=False)

    @property
    def token_parts(self):
        return self._parts


def chain_tokens(*parts):
    return TokenChain(*parts)


def token_parts(seq):
    """The ids of a token sequence as a list of 1-D numpy arrays, views where
    the source is a mapped buffer (the packer's part-wise read, loop.py:56-63)."""
    parts = getattr(seq, "token_parts", None)
    if parts is None:
        a = np.asarray(seq)
        return [a.reshape(-1)] if a.size else []
    out = []
    for part in parts:
        if isinstance(part, TokenView):
            out.append(part.numpy())
        elif isinstance(part, np.ndarray):
            out.append(part.reshape(-1))
        else:
            out.extend(token_parts(part))
    return out


def token_array(seq):
    """A sequence's token ids as one numpy array (tokens.py:495-511): the view
    itself for a single mapped part, else one concatenation; never a list."""
    parts = token_parts(seq)
    if not parts:
        return np.empty(0, dtype=np.int32)
    return parts[0] if len(parts) == 1 else np.concatenate(parts)


class ArrowTokenDocuments(_Rows):
    """A list<int> Arrow column as documents of TokenViews (tokens.py:103-136)."""

    def __init__(self, array):
        pieces = tuple(array.chunks) if hasattr(array, "chunks") else (array,)
        # document i lives in piece bisect(stops, i), at i - start of that piece
        self.stops = np.cumsum([len(c) for c in pieces], dtype=np.int64).tolist()
        self.piece_offsets = tuple(c.offsets.to_numpy(zero_copy_only=True) for c in pieces)
        self.piece_values = tuple(c.values for c in pieces)

    def __len__(self):
        return self.stops[-1] if self.stops else 0

    def row(self, i):
        c = bisect.bisect_right(self.stops, i)
        local = i - (self.stops[c - 1] if c else 0)
        offs = self.piece_offsets[c]
        lo, hi = int(offs[local]), int(offs[local + 1])
        return TokenView(self.piece_values[c].slice(lo, hi - lo))


# ------------------------------------------------------------- on-disk stores

def _pa():
    import pyarrow as pa
    return pa


class TokenLengths(_Rows):
    """A token store's document lengths, read from its count column (tokens.py:139-152)."""

    def __init__(self, store):
        self.store = store

    def __len__(self):
        return len(self.store)

    def row(self, i):
        b, local = self.store._locate(i)
        return int(self.store._counts[b][local])

    def numpy(self):
        """All lengths as one int64 array."""
        if not self.store._counts:
            return np.empty(0, dtype=np.int64)
        return np.concatenate(self.store._counts).astype(np.int64, copy=False)


def _token_schema(list_type):
    """The token store schema: ids and counts per document, tagged token_store."""
    pa = _pa()
    return pa.schema([pa.field(TokenStore.TOKEN_COLUMN, list_type, nullable=False),
                      pa.field(TokenStore.COUNT_COLUMN, pa.int64(), nullable=False)],
                     metadata={b"quail.kind": b"token_store"})


def _token_arrays(documents, list_type):
    """One record batch's columns for tokenized documents: the ids as one
    large_list array built from offsets over the concatenated ids, and the
    per-document counts."""
    pa = _pa()
    counts = np.fromiter(map(len, documents), dtype=np.int64, count=len(documents))
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    value_type = list_type.value_type
    flat = np.empty(int(offsets[-1]), dtype=value_type.to_pandas_dtype())
    for doc, lo, hi in zip(documents, offsets[:-1], offsets[1:]):
        flat[lo:hi] = token_array(doc)
    ids = pa.LargeListArray.from_arrays(pa.array(offsets), pa.array(flat, value_type))
    return [ids, pa.array(counts)]


class _IpcOutput:
    """A new Arrow IPC file taking record batches of one schema.

    seal() finishes the file (the footer makes it readable); discard()
    finishes and deletes it. Each may be called more than once; only the
    first call of either closes the file.
    """

    def __init__(self, path, schema):
        pa = _pa()
        self.path = path
        self.schema = schema
        self._file = pa.OSFile(path, "wb")
        self._batches = pa.ipc.new_file(self._file, schema)
        self.sealed = False

    def append(self, columns):
        batch = _pa().RecordBatch.from_arrays(list(columns), schema=self.schema)
        self._batches.write_batch(batch)

    def seal(self):
        if not self.sealed:
            self.sealed = True
            self._batches.close()
            self._file.close()

    def discard(self):
        self.seal()
        if os.path.exists(self.path):
            os.remove(self.path)


@contextlib.contextmanager
def _new_ipc_file(path, schema):
    """`with _new_ipc_file(path, schema) as out:` appends batches to a new
    file, sealed when the block ends and deleted if it raises, so a failed
    write never leaves a partial store behind."""
    out = _IpcOutput(path, schema)
    try:
        yield out
    except BaseException:
        out.discard()
        raise
    out.seal()


class TokenStoreWriter:
    """Tokenize the document column of source batches into a token store
    file, one record batch per source batch (tokens.py:193-229): the
    streaming form the session's scan uses; TokenStore.write runs it over
    a batch sequence."""

    def __init__(self, path, *, document_column, tokenizer, token_type):
        self.path = path
        self.document_column = document_column
        self.tokenizer = tokenizer
        self.list_type = _pa().large_list(token_type)
        self._out = _IpcOutput(path, _token_schema(self.list_type))

    def write_tokens(self, documents):
        """Append one batch of already tokenized documents (sequences of ids)."""
        self._out.append(_token_arrays(documents, self.list_type))

    def write_batch(self, batch):
        """Tokenize the document column of one source record batch."""
        texts = batch.column(self.document_column).to_pylist()
        self.write_tokens([self.tokenizer(text) for text in texts])

    def abort(self):
        """Close and delete the partial file."""
        self._out.discard()

    def finish(self):
        """Seal the file and open it as a TokenStore."""
        self._out.seal()
        return TokenStore(self.path)


class TokenStore:
    """Random access to the documents of one memory mapped token store file
    (tokens.py:296-356)."""

    TOKEN_COLUMN = "__quail_token_ids"
    COUNT_COLUMN = "__quail_token_count"

    def __init__(self, path):
        pa = _pa()
        self.path = path
        self._source = pa.memory_map(path, "r")
        self._reader = pa.ipc.open_file(self._source)
        self._docs, self._counts, self._ends = [], [], []
        total = 0
        for b in range(self._reader.num_record_batches):
            batch = self._reader.get_batch(b)
            self._docs.append(ArrowTokenDocuments(batch.column(self.TOKEN_COLUMN)))
            self._counts.append(batch.column(self.COUNT_COLUMN).to_numpy(zero_copy_only=True))
            total += batch.num_rows
            self._ends.append(total)
        self._lengths = TokenLengths(self)

    @classmethod
    def write(cls, path, batches, *, document_column, tokenizer, token_type):
        """Tokenize bounded source batches into one file and open it."""
        list_type = _pa().large_list(token_type)
        with _new_ipc_file(path, _token_schema(list_type)) as out:
            for batch in batches:
                texts = batch.column(document_column).to_pylist()
                out.append(_token_arrays([tokenizer(t) for t in texts], list_type))
        return cls(path)

    @classmethod
    def from_documents(cls, path, documents, *, token_type=None, batch_rows=4096):
        """Write already tokenized documents (sequences of ids), `batch_rows` per
        record batch, and open the file."""
        list_type = _pa().large_list(_pa().int32() if token_type is None else token_type)
        with _new_ipc_file(path, _token_schema(list_type)) as out:
            for start in range(0, len(documents), batch_rows):
                out.append(_token_arrays(documents[start:start + batch_rows], list_type))
        return cls(path)

    @property
    def lengths(self):
        return self._lengths

    def _locate(self, index):
        if index < 0:
            index += len(self)
        if not 0 <= index < len(self):
            raise IndexError(index)
        b = bisect.bisect_right(self._ends, index)
        return b, index - (self._ends[b - 1] if b else 0)

    def __len__(self):
        return self._ends[-1] if self._ends else 0

    def __getitem__(self, index):
        if isinstance(index, slice):
            return [self[i] for i in range(*index.indices(len(self)))]
        b, local = self._locate(index)
        return self._docs[b][local]

    def select(self, indices):
        return TokenSelection(self.path, indices)

    def flat_tokens(self):
        """Every document's ids as (ids, offsets) over one buffer: the mapped
        values themselves when the file holds one record batch, else one
        concatenation of the batches' values."""
        parts, offsets, base = [], [np.zeros(1, dtype=np.int64)], 0
        for docs in self._docs:
            for offs, values in zip(docs.piece_offsets, docs.piece_values):
                lo, hi = int(offs[0]), int(offs[-1])
                parts.append(values.to_numpy(zero_copy_only=True)[lo:hi])
                offsets.append(offs[1:].astype(np.int64) - lo + base)
                base += hi - lo
        if not parts:
            return np.empty(0, dtype=np.int32), offsets[0]
        if len(parts) == 1:
            ids = parts[0]
        else:
            wide = any(p.dtype != np.int32 for p in parts)
            ids = np.concatenate([p.astype(np.int64 if wide else np.int32, copy=False)
                                  for p in parts])
        return ids, np.concatenate(offsets)

    def close(self):
        self._source.close()


class ColumnStoreWriter:
    """Copy one source column into a column store file (tokens.py:232-251),
    batch by batch; ColumnStore.write runs it over a batch sequence."""

    def __init__(self, path, field):
        self.path = path
        self.name = field.name
        self._out = _IpcOutput(path, _pa().schema(
            [field], metadata={b"quail.kind": b"column_store"}))

    def write_batch(self, batch):
        self._out.append([batch.column(self.name)])

    def abort(self):
        self._out.discard()

    def finish(self):
        self._out.seal()
        return ColumnStore(self.path)


class ColumnStore:
    """One source column kept for result rows (tokens.py:254-287): the file is
    memory mapped and read as one table, so `values` is a chunked array over
    the mapped buffers (one chunk per record batch), never a copy."""

    def __init__(self, path):
        pa = _pa()
        self.path = path
        self._map = pa.memory_map(path, "r")
        table = pa.ipc.open_file(self._map).read_all()
        self.schema = table.schema
        self.name = table.schema.names[0]
        self.values = table.column(0)

    @classmethod
    def write(cls, path, batches, field):
        """Copy one column of bounded input batches into a file and open it."""
        schema = _pa().schema([field], metadata={b"quail.kind": b"column_store"})
        with _new_ipc_file(path, schema) as out:
            for batch in batches:
                out.append([batch.column(field.name)])
        return cls(path)

    def __len__(self):
        return len(self.values)

    def close(self):
        self.values = None
        self._map.close()


class TokenSelection(_Rows):
    """Selected documents of a token store, the file mapped on first access.
    It pickles as the file's path and the selected indices, so a child
    process maps the file itself instead of receiving the tokens
    (tokens.py:384-409)."""

    def __init__(self, path, indices):
        self.path = path
        self.picked = np.asarray(indices, dtype=np.int64)
        self.mapped = None

    def __len__(self):
        return len(self.picked)

    def row(self, i):
        if self.mapped is None:
            self.mapped = TokenStore(self.path)
        return self.mapped[int(self.picked[i])]

    def __reduce__(self):
        return TokenSelection, (self.path, self.picked)


def select_documents(documents, indices):
    """Selected documents, by file reference for a token store (tokens.py:458-462)."""
    if isinstance(documents, TokenStore):
        return documents.select(indices)
    return [documents[i] for i in indices]
