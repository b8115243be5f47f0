"""Seeded filter / join / prefix-tree scenarios shared by the fixture
generator (make_loop_golden.py, which runs the reference's own loop) and
the test that replays them through quail_amd (test_golden_loop.py).

Everything here is plain Python: inputs are regenerated from the seeds, so
the fixtures hold only the reference's outputs.
"""

import random


def corpus(rng, n, vocab=50):
    """Documents sharing headers and extending one another (so the prefix
    tree borrows), with exact duplicates and branch-offs."""
    header = [rng.randrange(vocab) for _ in range(rng.choice((0, 5, 16, 20, 33)))]
    docs = []
    while len(docs) < n:
        trace = list(header)
        for _ in range(rng.randrange(1, 4)):
            trace = trace + [rng.randrange(vocab) for _ in range(rng.choice((1, 7, 16, 30)))]
            docs.append(list(trace))
            if rng.random() < 0.2:
                docs.append(list(trace))
            if rng.random() < 0.3 and len(trace) > 20:
                cut = rng.randrange(1, len(trace))
                docs.append(trace[:cut] + [vocab + rng.randrange(20)])
    docs = docs[:n]
    rng.shuffle(docs)
    return docs


def answer_bit(token, position):
    """The stand-in model's answer for a final row: a fixed function of the
    row's token id and position, so two loops that pack identical chunks
    read identical answers."""
    return int((int(token) * 7 + int(position) * 13) % 5 < 3)


FILTERS = [dict(name=f"filter_{path}_{seed}", path=path, seed=seed)
           for seed in range(3) for path in ("unified", "tree")]
JOINS = [dict(name=f"join_{path}_{seed}", path=path, seed=seed)
         for seed in range(2) for path in ("unified", "tree")]
TREES = [dict(name=f"tree_{seed}", seed=seed) for seed in range(3)]


def filter_inputs(seed):
    rng = random.Random(1000 + seed)
    docs = corpus(rng, 26)
    n_stages = 1 + seed % 2
    preamble = [90, 91] if n_stages > 1 else []
    questions = [preamble + [92 + j, 93 + j, 94 + j][: 1 + (j + seed) % 3] for j in range(n_stages)]
    longest = max(map(len, docs)) + max(map(len, questions))
    budget = longest + (40, 300, 900)[seed]
    pages = max(-(-(max(map(len, docs)) + 16) // 16) * 3, (30, 60, 200)[seed])
    return docs, questions, budget, pages


def join_inputs(seed):
    rng = random.Random(2000 + seed)
    root = [rng.randrange(50) for _ in range(20 + 13 * seed)]
    anchors = [root + [rng.randrange(50) for _ in range(rng.randrange(1, 40))] for _ in range(9)]
    anchors.append(list(anchors[0]))
    frame = [95, 96, 97][: 2 + seed]
    partners = [[98] + [rng.randrange(50) for _ in range(rng.randrange(1, 12))] for _ in range(7)]
    n_stages = 1 + seed
    budget = max(map(len, anchors)) + len(frame) + max(map(len, partners)) + (20, 120)[seed]
    pages = (40, 120)[seed]
    return anchors, [list(frame)] * n_stages, [partners] * n_stages, budget, pages


def tree_inputs(seed):
    rng = random.Random(3000 + seed)
    docs = corpus(rng, 40, vocab=6 + seed)
    # exact duplicates and one-token tails: the tie order and the len-1 cap
    docs += [list(docs[0]), list(docs[1][:1]), [], list(docs[2]) + [0]]
    return docs
