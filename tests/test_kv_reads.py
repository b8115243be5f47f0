"""Every KV read of the filter loop is right, on seeded random corpora.

The reference runs the same kind of check over seeded corpora in
tests/test_kv_reads.py:24-148 and exhaustively over small documents in
tests/test_kv_reads_exhaustive.py:33-85. Documents here come in families
sharing random prefixes (so the prefix tree borrows pages), at budgets and
arena sizes small enough to force many chunks, page blocking and reuse.
"""

import itertools
import random

import pytest

from kv_checker import check_filter


def corpus(rng, n_docs, families, max_prefix, max_tail, vocab=50):
    heads = [[rng.randrange(vocab) for _ in range(rng.randrange(1, max_prefix))]
             for _ in range(families)]
    docs = []
    for _ in range(n_docs):
        head = rng.choice(heads)
        cut = rng.randrange(0, len(head) + 1)
        docs.append(head[:cut] + [rng.randrange(vocab) for _ in range(rng.randrange(1, max_tail))])
    return docs


@pytest.mark.parametrize("path", ["unified", "tree"])
@pytest.mark.parametrize("seed", range(6))
def test_filter_reads_over_random_corpora(path, seed):
    rng = random.Random(seed)
    docs = corpus(rng, rng.randrange(5, 40), rng.randrange(1, 5), 120, 80)
    n_stages = rng.randrange(1, 4)
    preamble = [rng.randrange(50) for _ in range(rng.randrange(0, 4))] if n_stages > 1 else []
    questions = [preamble + [rng.randrange(50) for _ in range(rng.randrange(1, 6))]
                 for _ in range(n_stages)]
    longest = max(map(len, docs)) + max(map(len, questions))
    budget = longest + rng.randrange(0, 400)
    pages = max(-(-(max(map(len, docs)) + 16) // 16) * 2, rng.randrange(20, 120))
    model, _ = check_filter(docs, questions, path=path, pages=pages, budget=budget)
    assert model.reads_checked > 0 or all(len(d) < 17 for d in docs)


@pytest.mark.parametrize("path", ["unified", "tree"])
def test_filter_reads_large_shared_prefix(path):
    # the AI.IF shape: every row = one 64-token instruction + its document
    rng = random.Random(99)
    instruction = [rng.randrange(1000) for _ in range(64)]
    docs = [instruction + [rng.randrange(1000) for _ in range(rng.randrange(1, 200))]
            for _ in range(60)]
    question = [[rng.randrange(1000) for _ in range(24)]]
    model, tokens = check_filter(docs, question, path=path, pages=400, budget=1500)
    # rows beyond the first computed only their own tokens
    assert tokens < sum(len(d) + 24 for d in docs) - 64 * 30


@pytest.mark.parametrize("path", ["unified", "tree"])
def test_filter_reads_every_pair_of_small_documents(path):
    # every ordered pair from a small alphabet of documents, tight budget
    alphabet = [[1] * 17, [1] * 16 + [2], [1] * 33, [3], [1] * 16 + [2] * 17]
    for a, b in itertools.product(alphabet, repeat=2):
        check_filter([a, b], [[7, 8], [7, 9]], path=path, pages=8,
                     budget=max(len(a), len(b)) + 2)
