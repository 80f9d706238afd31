"""Tail and head of a served model, and greedy generation (the continuous-batch backend's token step).

* ``lm_head_logits`` / ``greedy_pick`` -- ``lm_head(norm(h))`` then ``argmax(-1)``
  (``phase0/specpipe.py:796-800``; the greedy branches of ``Sampler.sample_logits`` / ``accept``,
  ``phase0/specsample.py:78-100``): RMSNorm with the fp32 final-norm weight, a bf16 Linear (fp32
  accumulate, one rounding to bf16), and torch.argmax semantics -- the first index of the maximum.
* ``embed`` -- ``parts["embed"](token_ids)`` (``specpipe.py:595-596``): a row gather.
* ``greedy_continue`` -- the oracle model (embed -> layer.stage_step -> tail) run teacher-forced over
  a whole token sequence, returning every position's logits, so a served generation can be checked
  position by position.

Parity: ``greedy_pick`` is pinned by a brute-force first-max loop and by exact small-integer logits;
``lm_head_logits`` reuses ``layer.rmsnorm`` / ``layer.linear`` (pinned against transformers)."""
import numpy as np
import torch

from . import layer
from .numerics import bf16


def embed(table, ids):
    return torch.as_tensor(table).float()[torch.as_tensor(np.asarray(ids, dtype=np.int64))]


def logits_from_normed(xn, lm_w):
    """bf16 Linear without bias: bf16(xn . W^T), accumulated in fp64 and rounded once."""
    w = torch.as_tensor(lm_w).double()
    return bf16((torch.as_tensor(xn).double() @ w.T).float())


def lm_head_logits(h, norm_w, lm_w, eps=layer.EPS):
    """h bf16-valued [R, H] (stage output rows) -> bf16-valued fp32 logits [R, V]."""
    return logits_from_normed(layer.rmsnorm(h, norm_w, eps), lm_w)


def greedy_pick(logits):
    """Row-wise first index of the maximum (torch.argmax semantics)."""
    lg = np.asarray(logits, dtype=np.float32)
    return lg.argmax(axis=-1).astype(np.int64)


def greedy_continue(ids, embed_w, layers, norm_w, lm_w, cos_tab, sin_tab, n_kv_heads=layer.N_KV_HEADS,
                    head_dim=layer.HEAD_DIM):
    """Teacher-forced pass over the sequence ``ids`` (one prefill from position 0): logits [L, V]."""
    L = len(ids)
    h = embed(embed_w, ids)
    kv = [([torch.zeros(n_kv_heads, L, head_dim)], [torch.zeros(n_kv_heads, L, head_dim)]) for _ in layers]
    h = layer.stage_step(h, layers, kv, [L], [0], cos_tab, sin_tab)
    return lm_head_logits(h, norm_w, lm_w)
