"""Prefix tree and sizing formulas against the reference's known answers.

prefix_tree: the known answers of tests/test_tokens.py:74-108 of the
reference and the worked example of docs/content/docs/architecture/
prefix-caching.mdx:38-50, as data (tests/golden/prefix_tree_cases.json).
Budgets: tests/test_specs_budgets.py:16-43 and tests/test_model_pipelines.py:
45-58 of the reference, and the MI355X sizing they imply.
"""

import json
import os
from dataclasses import replace

import numpy as np
import pytest

from quail_amd import budgets
from quail_amd.specs import H100_SXM, MI355X, QWEN3_4B_FP8, QWEN3_32B_FP8
from quail_amd.tokens import DocumentPrefixes, _prefix_tree_items, flat_tokens, prefix_tree

HERE = os.path.dirname(os.path.abspath(__file__))
TREE_CASES = json.load(open(os.path.join(HERE, "golden", "prefix_tree_cases.json")))["cases"]


def _document(runs):
    ids = []
    for kind, x, y in runs:
        ids.extend(range(x, y) if kind == "range" else [x] * y)
    return ids


@pytest.mark.parametrize("case", TREE_CASES, ids=[c["name"] for c in TREE_CASES])
def test_prefix_tree_known_answers(case):
    docs = [_document(runs) for runs in case["documents"]]
    tree = prefix_tree(docs, case["page_tokens"])
    for field in ("order", "parent", "shared", "shared_tokens"):
        if field in case:
            assert getattr(tree, field) == case[field], (case["name"], field)
    # parents come before their children in the order
    first = {doc: i for i, doc in enumerate(tree.order)}
    assert all(p is None or first[p] < first[d] for d, p in enumerate(tree.parent))


def test_worked_example_computes_each_token_once():
    """prefix-caching.mdx:38-50: three traces of one log, 1,000 / 1,400 /
    1,900 tokens, compute 1,000 + 408 + 508 tokens with borrowing."""
    case = next(c for c in TREE_CASES if c["name"] == "docs_worked_example")
    docs = [_document(runs) for runs in case["documents"]]
    tree = prefix_tree(docs, 16)
    assert sum(len(d) - s for d, s in zip(docs, tree.shared)) == 1000 + 408 + 508


def test_prefix_tree_sorts_ids_as_big_endian_int32():
    # 256 sorts after 1 even though its low byte is 0
    tree = prefix_tree([[256, 5], [1, 9], [255, 0]], 16)
    assert tree.order == [1, 2, 0]


def test_prefix_tree_orders_by_unsigned_big_endian_bytes():
    """Negative ids and ids of 2^31 and up sort by their int32 bytes read as
    unsigned big-endian numbers: 0 < 5 < 2^31 (0x80000000) < -1 (0xFFFFFFFF);
    a proper prefix sorts before its extensions, equal documents keep their
    input order."""
    tree = prefix_tree([[-1], [5], [2**31], [0], [5, 0], [5]], 16)
    assert tree.order == [3, 1, 5, 4, 2, 0]
    tree = prefix_tree(np.array([[-1], [5], [2**31], [0]], dtype=np.int64).tolist(), 16)
    assert tree.order == [3, 1, 2, 0]


def test_prefix_tree_of_words_sorts_them_as_tuples():
    """Tokens that are not integers (a test tokenizer's words) take the
    tuple order and item-by-item common prefix (tokens.py:556-564)."""
    words = [["b"] * 20, ["a"] * 20, ["a"] * 17 + ["c"]]
    tree = prefix_tree(words, 16)
    assert tree.order == [1, 2, 0]
    assert tree.parent == [None, None, 1] and tree.shared == [0, 0, 16]


@pytest.mark.parametrize("seed", range(6))
def test_native_prefix_tree_matches_the_item_restatement(seed):
    """Random documents over a small alphabet (long shared prefixes,
    duplicates, empty documents, pages of 1, 4 and 16): the host library's
    tree equals the pure-Python one on the same ids, int32 and int64, as
    lists and as one flat buffer."""
    rng = np.random.default_rng(seed)
    stems = [rng.integers(0, 3, size=int(rng.integers(0, 70))) for _ in range(6)]
    docs = []
    for _ in range(120):
        stem = stems[int(rng.integers(0, len(stems)))]
        cut = int(rng.integers(0, stem.size + 1))
        docs.append(np.concatenate([stem[:cut], rng.integers(0, 3, size=int(rng.integers(0, 20)))]))
    for page in (1, 4, 16):
        want = _prefix_tree_items([d.tolist() for d in docs], page)
        for dtype in (np.int32, np.int64):
            got = prefix_tree([d.astype(dtype) for d in docs], page)
            assert (got.order, got.parent, got.shared) == (want.order, want.parent, want.shared)


def test_flat_tokens_with_a_prefix_equals_the_rows():
    rng = np.random.default_rng(3)
    docs = [rng.integers(0, 1000, size=int(rng.integers(0, 9)), dtype=np.int32)
            for _ in range(50)]
    for prefix in ([], [7, 8, 9], np.array([2**31 + 1], dtype=np.int64)):
        ids, offsets = flat_tokens(docs, prefix)
        assert offsets[0] == 0 and offsets.size == len(docs) + 1
        for i, d in enumerate(docs):
            want = np.concatenate([np.asarray(prefix, dtype=np.int64), d.astype(np.int64)])
            assert np.array_equal(ids[offsets[i]:offsets[i + 1]].astype(np.int64), want)
        assert ids.dtype == (np.int64 if np.max(np.asarray(prefix, dtype=np.int64),
                                                initial=0) >= 2**31 else np.int32)
    ids, offsets = flat_tokens([], [1, 2])
    assert ids.size == 0 and offsets.tolist() == [0]


def test_document_prefixes_prepend_the_instruction():
    rows = DocumentPrefixes([7, 8], [[1, 2, 3], [4]])
    assert [list(r) for r in rows] == [[7, 8, 1, 2, 3], [7, 8, 4]]


def test_budgets_match_the_reference_on_h100_and_size_mi355x():
    assert QWEN3_4B_FP8.head_mem_bytes == 0.0
    assert QWEN3_32B_FP8.head_mem_bytes == 151_936 * 5_120 * 2
    tokens = budgets.arena_tokens(QWEN3_4B_FP8, H100_SXM)
    assert tokens == 362_240 and tokens // 16 == 22_640
    grown = budgets.arena_tokens(QWEN3_32B_FP8, H100_SXM)
    assert grown == 112_304
    kept = replace(QWEN3_32B_FP8, tied_head=True)
    assert grown - budgets.arena_tokens(kept, H100_SXM) == 5_936
    assert budgets.kernel_index_cap(QWEN3_4B_FP8) == (2**31 - 1) // 19456 == 110_376
    # MI355X: 288 GB HBM, 8 TB/s, fp8 5.03 PF
    assert budgets.chunk_budget(QWEN3_4B_FP8, MI355X) == 110_376
    assert budgets.arena_pages(QWEN3_4B_FP8, MI355X) == (106_394, 0)
    assert budgets.chunk_budget(QWEN3_32B_FP8, MI355X) == 41_943
    assert budgets.arena_pages(QWEN3_32B_FP8, MI355X) == (54_131, 0)
    assert abs(QWEN3_4B_FP8.gemm_flops_per_token() - 7.2666e9) < 1e6


def test_attention_path_choice_follows_the_roofline():
    # C3: ~400 readers of a 64-token node with ~250 rows each: unified
    assert budgets.choose_attention_path(QWEN3_4B_FP8, MI355X, readers=400,
                                         reader_rows=250, node_tokens=64) == "unified"
    # many short readers of a long node: tree
    assert budgets.choose_attention_path(QWEN3_4B_FP8, MI355X, readers=256,
                                         reader_rows=8, node_tokens=2048) == "tree"
    assert budgets.choose_attention_path(QWEN3_4B_FP8, MI355X, readers=1,
                                         reader_rows=8, node_tokens=2048) == "unified"
