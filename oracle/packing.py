"""Ragged batch packing (row a1), integer closed form, numpy.

The reference has no flat token tensor: ``BatchedFastVerify`` takes a rectangular h[B, kp1, H] and
derives per-stream positions as ``starts[:, None] + arange(kp1)`` (``phase0/batchverify.py:152-153``)
and the additive mask from ``_batched_causal_mask`` (``batchverify.py:51-61``; solo form
``phase0/pipeline.py:38-48``): query i of stream b sits at absolute position ``start_b + i`` and
attends key j iff ``j <= start_b + i`` and, on sliding layers, ``(start_b + i) - j < window``.
``FastVerify`` raises ``ContextOverflow`` before any write when ``start + q > maxlen``
(``phase0/fastverify.py:140-142``, ``:205-207``).

This restates that for variable per-sequence query lengths: decode rows (q=1), spec-verify rows
(q=K+1) and chunked-prefill rows (q=chunk) share one flat token axis.

Outputs, for S sequences and T = sum(q_lens) tokens:
  cu_seqlens int32[S+1]  exclusive prefix sum of q_lens (cu_seqlens[S] == T)
  positions  int32[T]    start_b + i for token i of sequence b
  seq_id     int32[T]    b
  kv_len     int32[S]    start_b + q_b (keys visible to the sequence's last token, inclusive)
  kv_slot    int64[T]    element offset of (kv head 0, position) in the KV pool:
                         kv_base[b] + positions * head_dim (head h adds h * kv_cap[b] * head_dim)

Parity: closed form; brute-force pure-Python loop in tests; the reference's own per-stream
position/mask equality (``tests/test_graph_batch.py:38-55``) is restated as a mask test.
"""
import numpy as np


class ContextOverflow(Exception):
    """A sequence needs more KV positions than its workspace holds (``fastverify.py:23-26``)."""


def pack_ragged(q_lens, starts, kv_base=None, kv_cap=None, head_dim=64):
    q_lens = np.asarray(q_lens, dtype=np.int64)
    starts = np.asarray(starts, dtype=np.int64)
    S = q_lens.shape[0]
    if starts.shape != (S,):
        raise ValueError("starts must have one entry per sequence")
    if np.any(q_lens < 1) or np.any(starts < 0):
        raise ValueError("q_lens must be >= 1 and starts >= 0")
    kv_len = starts + q_lens
    if kv_cap is not None:
        kv_cap = np.asarray(kv_cap, dtype=np.int64)
        bad = np.nonzero(kv_len > kv_cap)[0]
        if bad.size:
            b = int(bad[0])
            raise ContextOverflow(f"sequence {b} needs {int(kv_len[b])} positions > capacity {int(kv_cap[b])}")
    cu = np.zeros(S + 1, dtype=np.int64)
    cu[1:] = np.cumsum(q_lens)
    T = int(cu[-1])
    seq_id = np.repeat(np.arange(S, dtype=np.int64), q_lens)
    positions = starts[seq_id] + (np.arange(T, dtype=np.int64) - cu[seq_id])
    if kv_base is None:
        kv_base = np.zeros(S, dtype=np.int64)
    kv_base = np.asarray(kv_base, dtype=np.int64)
    kv_slot = kv_base[seq_id] + positions * head_dim
    return dict(cu_seqlens=cu.astype(np.int32), positions=positions.astype(np.int32),
                seq_id=seq_id.astype(np.int32), kv_len=kv_len.astype(np.int32),
                kv_slot=kv_slot.astype(np.int64))


def allowed_keys(position, window):
    """Half-open key interval [lo, hi) a query at absolute ``position`` attends (pipeline.py:38-48)."""
    lo = 0 if not window else max(0, position - window + 1)
    return lo, position + 1


def batched_mask(q_lens, starts, alen, window):
    """Dense boolean [T, alen] allow-mask in packed-token order; the pure restatement of
    ``_batched_causal_mask`` (batchverify.py:51-61) generalised to ragged q."""
    p = pack_ragged(q_lens, starts)
    rows = p["positions"].astype(np.int64)[:, None]
    cols = np.arange(alen, dtype=np.int64)[None, :]
    allow = cols <= rows
    if window:
        allow &= (rows - cols) < window
    return allow
