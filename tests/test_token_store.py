"""Token store files (Arrow IPC, memory mapped) and the token views the
packer reads from them (quail/execution/tokens.py:13-152, :164-409).

The file layout is the reference's, checked column by column against a
file written with plain pyarrow; documents read back are views into the
mapped buffer; and the golden filter / join scenarios, run from documents
stored in a token store, still pack the reference's chunks bit for bit.
"""

import os
import pickle
import random
import sys

import numpy as np
import pyarrow as pa
import pytest
import torch

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, HERE)
import scenarios  # noqa: E402
from replay import Passthrough, Recorder, arena, compare  # noqa: E402

from quail_amd import loop  # noqa: E402
from quail_amd.aiif import RowPrompts  # noqa: E402
from quail_amd.tokens import (ColumnStore, TokenChain, TokenSelection, TokenStore,  # noqa: E402
                              TokenView, chain_tokens, prefix_tree, select_documents,
                              token_array, token_parts)


def _docs(seed, n=40, vocab=151_936):
    rng = np.random.default_rng(seed)
    return [rng.integers(0, vocab, size=int(rng.integers(0, 60)), dtype=np.int64)
            for _ in range(n)]


@pytest.mark.parametrize("token_type", [pa.int32(), pa.int64()])
def test_round_trip_over_several_record_batches(tmp_path, token_type):
    docs = _docs(1)
    store = TokenStore.from_documents(str(tmp_path / "t.arrow"), docs, token_type=token_type,
                                      batch_rows=7)
    assert store._reader.num_record_batches == 6
    assert len(store) == len(docs)
    assert list(store.lengths) == [len(d) for d in docs]
    assert np.array_equal(store.lengths.numpy(), [len(d) for d in docs])
    for i, d in enumerate(docs):
        got = store[i]
        assert isinstance(got, TokenView) and len(got) == len(d)
        assert np.array_equal(got.numpy(), d)
        if len(d) > 3:
            assert got[2] == int(d[2]) and got[-1] == int(d[-1])
            assert np.array_equal(got[1:-1].numpy(), d[1:-1])
    assert np.array_equal(store[-1].numpy(), docs[-1])
    with pytest.raises(IndexError):
        store[len(docs)]
    assert [len(v) for v in store[3:9]] == [len(d) for d in docs[3:9]]


def test_layout_is_the_reference_token_store(tmp_path):
    """Column names, types, nullability and metadata as tokens.py:193-210 /
    :316-319 write them; a file built directly with pyarrow in that layout
    reads back through TokenStore."""
    docs = _docs(2, n=9)
    store = TokenStore.from_documents(str(tmp_path / "ours.arrow"), docs, batch_rows=4)
    schema = store._reader.schema
    assert schema.names == ["__quail_token_ids", "__quail_token_count"]
    assert schema.field(0).type == pa.large_list(pa.int32()) and not schema.field(0).nullable
    assert schema.field(1).type == pa.int64() and not schema.field(1).nullable
    assert schema.metadata == {b"quail.kind": b"token_store"}

    path = str(tmp_path / "plain.arrow")
    plain = pa.schema([pa.field("__quail_token_ids", pa.large_list(pa.int32()), nullable=False),
                       pa.field("__quail_token_count", pa.int64(), nullable=False)],
                      metadata={b"quail.kind": b"token_store"})
    with pa.OSFile(path, "wb") as sink, pa.ipc.new_file(sink, plain) as w:
        for lo in (0, 5):
            part = [d.astype(np.int32).tolist() for d in docs[lo:lo + 5]]
            w.write_batch(pa.RecordBatch.from_arrays(
                [pa.array(part, type=pa.large_list(pa.int32())),
                 pa.array([len(p) for p in part], type=pa.int64())], schema=plain))
    other = TokenStore(path)
    assert len(other) == len(docs)
    for i, d in enumerate(docs):
        assert np.array_equal(other[i].numpy(), d)
        assert other.lengths[i] == len(d)


def test_documents_are_views_of_the_mapped_file(tmp_path):
    """No copy on read: a document's ids are the mapped values buffer at the
    document's offset."""
    docs = [np.arange(10 * i, 10 * i + 10, dtype=np.int32) for i in range(6)]
    store = TokenStore.from_documents(str(tmp_path / "t.arrow"), docs)
    a, b = store[1].numpy(), store[2].numpy()
    assert not a.flags.owndata and not a.flags.writeable
    values = store[1].arrow_array
    base = values.buffers()[1].address + values.offset * 4
    assert a.__array_interface__["data"][0] == base
    assert b.__array_interface__["data"][0] - a.__array_interface__["data"][0] == 40
    # a chain of one mapped part hands that part back without copying
    assert token_array(chain_tokens(store[3])).__array_interface__["data"][0] == \
        store[3].numpy().__array_interface__["data"][0]


def test_chains_slice_and_read_like_one_array():
    rng = random.Random(5)
    for _ in range(200):
        pieces = [np.array([rng.randrange(1000) for _ in range(rng.randrange(0, 6))],
                           dtype=np.int64) for _ in range(rng.randrange(1, 5))]
        whole = np.concatenate(pieces)
        chain = TokenChain(*pieces[:1], TokenChain(*pieces[1:]))
        assert len(chain) == whole.size
        assert all(len(p) for p in chain.token_parts)
        assert np.array_equal(np.asarray(chain), whole)
        assert list(chain) == whole.tolist()
        if whole.size:
            i = rng.randrange(-whole.size, whole.size)
            assert chain[i] == whole[i]
        lo, hi = sorted((rng.randrange(whole.size + 1), rng.randrange(whole.size + 1)))
        assert np.array_equal(np.asarray(chain[lo:hi], dtype=np.int64), whole[lo:hi])
        assert sum(p.size for p in token_parts(chain[lo:hi])) == hi - lo
    with pytest.raises(IndexError):
        TokenChain(np.arange(3))[3]


def test_selection_pickles_as_a_file_reference(tmp_path):
    docs = _docs(3, n=12)
    store = TokenStore.from_documents(str(tmp_path / "t.arrow"), docs, batch_rows=5)
    sel = select_documents(store, [7, 2, 11])
    assert isinstance(sel, TokenSelection)
    blob = pickle.dumps(sel)
    assert len(blob) < 300                     # the path and the indices only
    back = pickle.loads(blob)
    for j, i in enumerate([7, 2, 11]):
        assert np.array_equal(back[j].numpy(), docs[i])
    assert [np.asarray(d).tolist() for d in select_documents(docs, [1, 0])] == \
        [docs[1].tolist(), docs[0].tolist()]


def test_column_store_round_trip(tmp_path):
    field = pa.field("title", pa.string())
    batches = [pa.RecordBatch.from_arrays([pa.array(["a", "bb"]), pa.array([1, 2])],
                                          names=["title", "n"]),
               pa.RecordBatch.from_arrays([pa.array(["ccc"]), pa.array([3])],
                                          names=["title", "n"])]
    col = ColumnStore.write(str(tmp_path / "c.arrow"), batches, field)
    assert col.name == "title" and len(col) == 3
    assert col.values.to_pylist() == ["a", "bb", "ccc"]
    assert col.schema.metadata == {b"quail.kind": b"column_store"}
    assert pa.ipc.open_file(str(tmp_path / "c.arrow")).schema.metadata == \
        {b"quail.kind": b"column_store"}


def test_writer_tokenizes_a_document_column(tmp_path):
    batches = [pa.RecordBatch.from_arrays([pa.array(["ab", "c", ""])], names=["text"])]
    store = TokenStore.write(str(tmp_path / "t.arrow"), batches, document_column="text",
                             tokenizer=lambda s: [ord(ch) for ch in s],
                             token_type=pa.int32())
    assert [np.asarray(store[i]).tolist() for i in range(3)] == [[97, 98], [99], []]


def test_streaming_writers_finish_and_abort(tmp_path):
    """The session's route (quail/execution/session.py:473-501): one writer per
    stored column, a batch at a time, finish() opening the store and abort()
    removing the partial file."""
    from quail_amd.tokens import ColumnStoreWriter, TokenStoreWriter
    batches = [pa.RecordBatch.from_arrays([pa.array(["ab", ""]), pa.array([7, 8])],
                                          names=["text", "n"]),
               pa.RecordBatch.from_arrays([pa.array(["xyz"]), pa.array([9])],
                                          names=["text", "n"])]
    tw = TokenStoreWriter(str(tmp_path / "t.arrow"), document_column="text",
                          tokenizer=lambda s: [ord(ch) for ch in s], token_type=pa.int64())
    cw = ColumnStoreWriter(str(tmp_path / "n.arrow"), pa.field("n", pa.int64()))
    for b in batches:
        tw.write_batch(b)
        cw.write_batch(b)
    store, col = tw.finish(), cw.finish()
    assert [np.asarray(store[i]).tolist() for i in range(3)] == [[97, 98], [], [120, 121, 122]]
    assert store.lengths.numpy().tolist() == [2, 0, 3]
    assert col.values.to_pylist() == [7, 8, 9] and col.values.num_chunks == 2
    for cls, kw in ((TokenStoreWriter, dict(document_column="text", tokenizer=list,
                                            token_type=pa.int32())),
                    (ColumnStoreWriter, dict(field=pa.field("n", pa.int64())))):
        path = str(tmp_path / "partial.arrow")
        w = cls(path, **kw)
        assert os.path.exists(path)
        w.abort()
        w.abort()
        assert not os.path.exists(path)


def test_failed_write_leaves_no_file(tmp_path):
    path = str(tmp_path / "t.arrow")

    def bad(_):
        raise RuntimeError("tokenizer failed")
    batches = [pa.RecordBatch.from_arrays([pa.array(["x"])], names=["text"])]
    with pytest.raises(RuntimeError):
        TokenStore.write(path, batches, document_column="text", tokenizer=bad,
                         token_type=pa.int32())
    assert not os.path.exists(path)


@pytest.mark.parametrize("sc", scenarios.TREES, ids=[s["name"] for s in scenarios.TREES])
def test_prefix_tree_of_a_token_store(tmp_path, sc):
    docs = scenarios.tree_inputs(sc["seed"])
    store = TokenStore.from_documents(str(tmp_path / "t.arrow"), docs, batch_rows=9)
    a, b = prefix_tree(docs, 16), prefix_tree(store, 16)
    assert (a.order, a.parent, a.shared) == (b.order, b.parent, b.shared)


@pytest.mark.parametrize("sc", scenarios.FILTERS, ids=[s["name"] for s in scenarios.FILTERS])
def test_filter_from_a_token_store_packs_the_reference_chunks(tmp_path, sc):
    docs, questions, budget, pages = scenarios.filter_inputs(sc["seed"])
    store = TokenStore.from_documents(str(tmp_path / "t.arrow"), docs, batch_rows=5)
    rec, stats = Recorder(), {}
    answers, _, total = loop.run_filter(
        torch, arena(pages), rec, Passthrough(), store, questions, budget, arena_writes=True,
        arena_keys=[("d", i) for i in range(len(store))], attention_mode=sc["path"],
        prefix_tree=prefix_tree(store, 16), stats=stats)
    want = compare(sc["name"], rec)
    assert {str(k): v for k, v in answers.items()} == want["answers"]
    assert total == want["tokens"] and stats["borrowed_tokens"] == want["borrowed"]


@pytest.mark.parametrize("sc", scenarios.JOINS, ids=[s["name"] for s in scenarios.JOINS])
def test_join_from_a_token_store_packs_the_reference_chunks(tmp_path, sc):
    anchors, frames, suffixes, budget, pages = scenarios.join_inputs(sc["seed"])
    store = TokenStore.from_documents(str(tmp_path / "t.arrow"), anchors, batch_rows=4)
    rec, stats = Recorder(), {}
    answers, _, total = loop.run_join(
        torch, arena(pages), rec, Passthrough(), store, suffixes, budget,
        stage_frames=frames, anchor_keys=[("a", i) for i in range(len(store))],
        attention_mode=sc["path"], prefix_tree=prefix_tree(store, 16), stats=stats)
    want = compare(sc["name"], rec)
    assert [{str(k): v for k, v in s.items()} for s in answers] == want["answers"]
    assert total == want["tokens"] and stats["borrowed_tokens"] == want["borrowed"]


@pytest.mark.parametrize("batch_rows,token_type", [(4096, None), (7, None), (5, "int64")])
def test_flat_tokens_of_a_store_and_its_row_prompts(tmp_path, batch_rows, token_type):
    """A store's flat buffer is its documents in order (the mapped values
    themselves for one record batch); RowPrompts over it adds the
    instruction to every row, and the packer's token table reads the same
    lengths from it."""
    docs = _docs(6, n=30)
    tt = None if token_type is None else pa.int64()
    store = TokenStore.from_documents(str(tmp_path / "t.arrow"), docs, batch_rows=batch_rows,
                                      token_type=tt)
    ids, offsets = store.flat_tokens()
    assert offsets.tolist() == np.concatenate([[0], np.cumsum([d.size for d in docs])]).tolist()
    assert np.array_equal(ids.astype(np.int64), np.concatenate(docs))
    if batch_rows >= len(docs) and token_type is None:
        assert np.shares_memory(ids, store[0].numpy())
    instruction = np.arange(4, dtype=np.int64) + 10
    rows = RowPrompts(instruction, store)
    ids, offsets = rows.flat_tokens()
    for i, d in enumerate(docs):
        assert np.array_equal(ids[offsets[i]:offsets[i + 1]].astype(np.int64),
                              np.concatenate([instruction, d]))
    assert rows.lengths().tolist() == [d.size + 4 for d in docs]
    table = loop.TokenTable(rows)
    assert [table.length(i) for i in range(len(docs))] == [d.size + 4 for d in docs]


def test_row_prompts_of_arrays_are_views_of_one_buffer(tmp_path):
    docs = _docs(8, n=12)
    instruction = np.array([5, 6], dtype=np.int64)
    rows = RowPrompts(instruction, docs)
    ids, offsets = rows.flat_tokens()
    for i, d in enumerate(docs):
        assert np.shares_memory(rows[i], ids) or rows[i].size == 0
        assert np.array_equal(rows[i], np.concatenate([instruction, d]))
    assert np.array_equal(rows[-1], rows[len(docs) - 1])
    with pytest.raises(IndexError):
        rows[len(docs)]
    # slices give lists of rows, as the list of rows this replaces did
    part = rows[2:5]
    assert isinstance(part, list) and len(part) == 3
    assert all(np.array_equal(a, rows[i]) for a, i in zip(part, range(2, 5)))
    # a token store of prompt rows reads back the same rows
    store = TokenStore.from_documents(str(tmp_path / "rows.arrow"), rows, batch_rows=5)
    assert len(store) == len(rows)
    assert all(np.array_equal(store[i].numpy(), rows[i]) for i in range(len(rows)))


def test_row_prompts_chain_stored_documents(tmp_path):
    """Rows over a token store are instruction + document chains over the
    mapped buffer (tokens.py:412-429), equal to the materialised rows."""
    docs = _docs(4, n=8)
    store = TokenStore.from_documents(str(tmp_path / "t.arrow"), docs)
    instruction = np.arange(5, dtype=np.int64)
    rows = RowPrompts(instruction, store)
    for i, d in enumerate(docs):
        assert isinstance(rows[i], TokenChain)
        assert np.array_equal(np.asarray(rows[i], dtype=np.int64), np.concatenate([instruction, d]))
