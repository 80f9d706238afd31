"""The tail's token sampler: temperature / top-k / top-p and lossless speculative-sampling acceptance.

Mirrors ``Sampler`` of ``phase0/specsample.py:36-107`` (same constructor, attribute and method names,
argument meaning): ``dist`` (filtered, renormalised distribution), ``sample`` (a draw from a
probability vector), ``uniform``, ``sample_logits`` (greedy argmax or one sampled token) and ``accept``
(the doctored result list r of length K+1 for a deterministic draft: accept d_j with probability
p_j(d_j), on the first rejection a draw from p_j with d_j removed, a bonus draw from p_K when all K
accept; greedy -> the argmax of every row).

The filtering and the draws run in ``flyai_sample_rows`` / ``flyai_sample_probs`` on the GPU over exact
integer weights w = floor(2^40 e^(z - max z)); only the uniforms come from the host: a numpy PCG64
generator seeded with ``seed``, so a run's receipts are reproducible (the reference seeds a torch
generator instead; its stream cannot be matched, and the distribution of every output is what the
accept rule preserves).  ``accept`` makes one launch for the K+1 drafted probabilities, one host copy,
and one launch for the residual or bonus draw."""
import numpy as np
import torch

from . import ops


class Sampler:
    """Temperature / top-k / top-p sampler with a seeded generator (reproducible receipts); temp <= 0
    is greedy (argmax of the logits)."""

    def __init__(self, temp=0.0, top_p=1.0, top_k=0, seed=0, device="cuda"):
        self.temp = float(temp)
        self.top_p = float(top_p)
        self.top_k = int(top_k)
        if self.top_k < 0:
            raise ValueError("top_k must be >= 0")
        self.greedy = self.temp <= 0.0
        self.device = torch.device(device)
        self.gen = np.random.Generator(np.random.PCG64(int(seed) & 0x7FFFFFFFFFFFFFFF))

    def _rows(self, logits):
        x = logits.to(self.device)
        if x.dtype != torch.bfloat16:
            raise TypeError(f"logits must be bfloat16 (the lm_head's output), got {x.dtype}")
        return x.reshape(-1, x.shape[-1]).contiguous()

    def dist(self, logits_row):
        """logits_row [V] bf16 -> [V] float32 probability vector on self.device (greedy: one-hot)."""
        x = self._rows(logits_row)
        return ops.sample_rows(x, self.temp, self.top_k, self.top_p, want_probs=True)["probs"][0]

    def sample(self, probs):
        """Draw one token id from a probability vector (already normalised)."""
        p = probs.to(self.device, torch.float32).contiguous()
        return int(ops.sample_probs(p, self.uniform()).item())

    def uniform(self):
        return float(self.gen.random())

    def sample_logits(self, logits_row):
        """One token from a single logits row: greedy -> argmax, else a temperature / top-k / top-p draw."""
        x = self._rows(logits_row)
        u = None if self.greedy else torch.tensor([self.uniform()], dtype=torch.float64, device=self.device)
        return int(ops.sample_rows(x, self.temp, self.top_k, self.top_p, u=u, want_draw=True)["draw"].item())

    def sample_logits_rows(self, logits):
        """``sample_logits`` of every row of logits [n, V] in one launch, consuming one uniform per row in
        row order (the same tokens as n calls of ``sample_logits``)."""
        x = self._rows(logits)
        if self.greedy:
            return ops.sample_rows(x, 0.0, want_draw=True)["draw"].tolist()
        u = torch.tensor([self.uniform() for _ in range(x.shape[0])], dtype=torch.float64, device=self.device)
        return ops.sample_rows(x, self.temp, self.top_k, self.top_p, u=u, want_draw=True)["draw"].tolist()

    def _draw_row(self, x, exclude):
        d = torch.tensor([exclude], dtype=torch.int32, device=self.device)
        u = torch.tensor([self.uniform()], dtype=torch.float64, device=self.device)
        return int(ops.sample_rows(x, self.temp, self.top_k, self.top_p, draft=d, u=u, want_draw=True)["draw"].item())

    def accept(self, logits, draft):
        """Speculative-sampling acceptance for a deterministic draft.  logits [K+1, V] bf16 (row j
        predicts the token after chunk slot j); draft: K ids.  Returns r (length K+1): greedy -> the
        argmax of every row; sampled -> r[j] = d_j for accepted slots, r[m] = the residual draw at the
        first rejection (never d_m), r[K] = the bonus draw when all K accept."""
        K = len(draft)
        x = self._rows(logits)
        if x.shape[0] != K + 1:
            raise ValueError(f"accept: {K} drafted tokens need {K + 1} logits rows, got {x.shape[0]}")
        if self.greedy:
            return ops.sample_rows(x, 0.0, want_draw=True)["draw"].tolist()
        V = x.shape[1]
        if any(not 0 <= int(d) < V for d in draft):
            raise ValueError("accept: drafted token id outside the vocabulary")
        d = torch.tensor(list(draft) + [-1], dtype=torch.int32, device=self.device)
        p = ops.sample_rows(x, self.temp, self.top_k, self.top_p, draft=d, want_p_draft=True)["p_draft"].tolist()
        r = [0] * (K + 1)
        for j in range(K):
            if self.uniform() < p[j]:
                r[j] = int(draft[j])
                continue
            r[j] = self._draw_row(x[j:j + 1], int(draft[j]))
            return r
        r[K] = self._draw_row(x[K:K + 1], -1)
        return r


def tail_tokens(parts, h, sampler, prefill=False, draft=None):
    """The tail's reply for one verify message (``phase0/specpipe.py:790-803``): h [1, n, H] is the last
    stage's output rows, ``parts`` holds ``norm`` and ``lm_head`` callables.  Prefill -> [one token from
    the last row]; no draft -> one token per row (greedy: the fused lm_head argmax when the head has one,
    so no logits are written); a draft of n - 1 ids -> ``sampler.accept`` over the n logits rows."""
    if prefill:
        h = h[:, -1:]
    x = parts["norm"](h)
    head = parts["lm_head"]
    if prefill:
        return [sampler.sample_logits(head(x)[0, -1])]
    if draft is None:
        if sampler.greedy and hasattr(head, "argmax"):
            return head.argmax(x)[0].tolist()
        return sampler.sample_logits_rows(head(x)[0])
    return sampler.accept(head(x)[0], list(draft))
