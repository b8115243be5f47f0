"""TRUE/FALSE readout of the answer rows (quail/backends/quail/executor/readout.py).

AnswerRows holds the retained output-head rows of the query's answer ids;
AsyncAnswers scores the final-normed rows on the GPU (one kernel: bf16
scores, per-class max, strict TRUE > FALSE, readout.py:45-49, :70-79) and
copies the bits into a reusable pinned slot without stalling the stream;
result() waits on that slot's copy.
"""

from quail_amd import kernels
from quail_amd.model import answer_weights


class AnswerRows:
    def __init__(self, torch, model, true_ids, false_ids):
        self.torch = torch
        true_ids, false_ids = set(true_ids), set(false_ids)
        self.allowed = sorted(true_ids | false_ids)
        self.weights = answer_weights(model, self.allowed)
        self.true_cols = [i for i, t in enumerate(self.allowed) if t in true_ids]
        self.false_cols = [i for i, t in enumerate(self.allowed) if t in false_ids]
        mask = [1 if t in true_ids else 0 for t in self.allowed]
        self.is_true = torch.tensor(mask, dtype=torch.uint8, device=self.weights.device)

    def logits(self, normed):
        """Per row, the best logit of each class over its spellings: bf16
        (best TRUE, best FALSE), as readout.py:45-49 returns them."""
        return kernels.answer_logits(normed, self.weights, self.is_true)

    def bits(self, normed, with_margin=False):
        return kernels.answer_bits(normed, self.weights, self.is_true, with_margin)

    def __call__(self, normed):
        bits, _ = self.bits(normed)
        return [int(b) for b in bits.cpu().tolist()]


class _PinnedSlot:
    """One in-flight readout: pinned host arrays that the chunk's bits (and
    margins) are copied into, and the event that marks the copy done. A slot
    keeps its arrays between uses and grows them only for a larger chunk."""

    def __init__(self, torch):
        self.torch = torch
        self.capacity = 0
        self.bits = self.margin = None
        self.rows = 0
        self.has_margin = False
        self.copied = torch.cuda.Event()

    def load(self, bits, margin):
        torch = self.torch
        n = bits.shape[0]
        if n > self.capacity:
            self.capacity = max(n, 2 * self.capacity)
            self.bits = torch.empty(self.capacity, dtype=torch.uint8, pin_memory=True)
            self.margin = torch.empty(self.capacity, dtype=torch.float32, pin_memory=True)
        self.rows = n
        self.bits[:n].copy_(bits, non_blocking=True)
        self.has_margin = margin is not None
        if self.has_margin:
            self.margin[:n].copy_(margin, non_blocking=True)
        self.copied.record()

    def unload(self):
        self.copied.synchronize()
        n = self.rows
        margin = self.margin[:n].numpy().copy() if self.has_margin else None
        return self.bits[:n].tolist(), margin


class AsyncAnswers:
    """Non-blocking TRUE/FALSE readout for AI_FILTER (readout.py:57-85).

    submit() launches the readout kernel, starts the copy of its bits into a
    pinned slot and returns the slot as the handle; result(handle) waits for
    that copy and returns the bits, and the slot goes back to the pool for a
    later chunk (a slot is reused only after its copy has been waited on).
    With keep_margins, result() also stores each row's logit margin (max TRUE
    - max FALSE) in self.margins, for decision-parity reports.
    """

    dtype = None

    def __init__(self, torch, rows, keep_margins=False):
        self.torch = torch
        self.rows = rows
        self.keep_margins = keep_margins
        self.margins = []
        self._idle = []

    def submit(self, normed):
        bits, margin = self.rows.bits(normed, with_margin=self.keep_margins)
        slot = self._idle.pop() if self._idle else _PinnedSlot(self.torch)
        slot.load(bits, margin)
        return slot

    def result(self, handle):
        bits, margin = handle.unload()
        self._idle.append(handle)
        if margin is not None:
            self.margins.append(margin)
        return bits
