"""TRUE/FALSE readout of the answer rows (quail/backends/quail/executor/readout.py).

AnswerRows holds the retained output-head rows of the query's answer ids;
AsyncAnswers scores the final-normed rows on the GPU (one kernel: bf16
scores, per-class max, strict TRUE > FALSE, readout.py:45-49, :70-79),
copies the bits to pinned host memory without stalling the stream, and
result() waits on that copy's event.
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

    def bits(self, normed, with_margin=False):
        return kernels.answer_bits(normed, self.weights, self.is_true, with_margin)

    def __call__(self, normed):
        bits, _ = self.bits(normed)
        return [int(b) for b in bits.cpu().tolist()]


class AsyncAnswers:
    """Non-blocking TRUE/FALSE readout for AI_FILTER (readout.py:57-85).

    With keep_margins, result() also stores each row's logit margin
    (max TRUE - max FALSE) in self.margins, for decision-parity reports.
    """

    dtype = None

    def __init__(self, torch, rows, keep_margins=False):
        self.torch = torch
        self.rows = rows
        self.keep_margins = keep_margins
        self.margins = []

    def submit(self, normed):
        torch = self.torch
        bits, margin = self.rows.bits(normed, with_margin=self.keep_margins)
        host = torch.empty(bits.shape[0], dtype=torch.uint8, pin_memory=True)
        host.copy_(bits, non_blocking=True)
        host_m = None
        if margin is not None:
            host_m = torch.empty(margin.shape[0], dtype=torch.float32, pin_memory=True)
            host_m.copy_(margin, non_blocking=True)
        event = torch.cuda.Event()
        event.record()
        return event, host, host_m

    def result(self, handle):
        event, host, host_m = handle
        event.synchronize()
        if host_m is not None:
            self.margins.append(host_m.numpy().copy())
        return [int(b) for b in host.tolist()]
