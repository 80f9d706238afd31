"""Ragged GQA attention with learned sinks and an optional sliding window (row a8).

Follows ``eager_attention_forward`` (``transformers/models/gpt_oss/modeling_gpt_oss.py:235-263``)
with the masks of ``phase0/pipeline.py:38-48`` / ``phase0/batchverify.py:51-61`` and the GQA head
map of ``repeat_kv`` (``modeling_gpt_oss.py:203-212``: query head h reads kv head h // n_rep):

    s_j   = (q . k_j) * head_dim**-0.5            for keys j in [lo(p), p], p = start_b + i
    m     = max(max_j s_j, sink_h)
    P_j   = exp(s_j - m) / (sum_j exp(s_j - m) + exp(sink_h - m))     (the sink column is dropped)
    o     = bf16(sum_j P_j v_j)

lo(p) = 0 on full layers and max(0, p - window + 1) on sliding layers.  Computed in fp32 (HF runs
the softmax in bf16; the bf16 rounding of probabilities is inside the tolerance bar).  Keys of
the current step are written into the cache before attention reads it (``fastverify.py:71-77``),
so the tokens of a verify or prefill chunk see each other causally.

Parity: pure-Python brute force on tiny shapes (tests), closed-form mask, and a transformers
fixture of ``eager_attention_forward`` with an additive mask (tests/golden).  ``tree_attention``
(tree verify) is pinned by fp64 brute force over the reference's dense tree mask and by the chain
tree, which must equal causal verify attention.
"""
import math

import numpy as np
import torch

from .numerics import bf16
from .packing import allowed_keys


def ragged_attention(q, k_seqs, v_seqs, q_lens, starts, sinks, window, scale=None):
    """q fp32 [T, Hq, D] (bf16 values); k_seqs[b] / v_seqs[b] fp32 [Hkv, >= start_b + q_b, D];
    sinks fp32 [Hq].  Returns bf16-valued fp32 [T, Hq, D] in packed token order."""
    q = torch.as_tensor(q).float()
    T, Hq, D = q.shape
    scale = D ** -0.5 if scale is None else scale
    sinks = torch.as_tensor(sinks).float()
    out = torch.zeros(T, Hq, D, dtype=torch.float32)
    t = 0
    for b, (ql, st) in enumerate(zip(q_lens, starts)):
        ql, st = int(ql), int(st)
        K = torch.as_tensor(k_seqs[b]).float()
        V = torch.as_tensor(v_seqs[b]).float()
        Hkv = K.shape[0]
        n_rep = Hq // Hkv
        hi_all = st + ql
        lo_all = allowed_keys(st, window)[0]
        kk = K[:, lo_all:hi_all, :]                                      # [Hkv, n, D]
        vv = V[:, lo_all:hi_all, :]
        qq = q[t:t + ql].view(ql, Hkv, n_rep, D).permute(1, 0, 2, 3)      # [Hkv, ql, n_rep, D]
        s = torch.einsum("gird,gnd->girn", qq, kk) * scale               # [Hkv, ql, n_rep, n]
        keys = torch.arange(lo_all, hi_all)
        allow = torch.zeros(ql, keys.numel(), dtype=torch.bool)
        for i in range(ql):
            lo, hi = allowed_keys(st + i, window)
            allow[i] = (keys >= lo) & (keys < hi)
        s = torch.where(allow[None, :, None, :], s, torch.tensor(float("-inf")))
        sk = sinks.view(Hkv, 1, n_rep, 1).expand(Hkv, ql, n_rep, 1)
        m = torch.maximum(s.amax(dim=-1, keepdim=True), sk)
        e = torch.exp(s - m)
        den = e.sum(dim=-1, keepdim=True) + torch.exp(sk - m)
        p = e / den
        o = torch.einsum("girn,gnd->gird", p, vv)                        # [Hkv, ql, n_rep, D]
        out[t:t + ql] = o.permute(1, 0, 2, 3).reshape(ql, Hq, D)
        t += ql
    return bf16(out)


def brute_force_attention(q, k_seqs, v_seqs, q_lens, starts, sinks, window, scale=None):
    """Pure-Python loop version (fp64) for tiny shapes; the independent check of the above."""
    q = np.asarray(q, dtype=np.float64)
    T, Hq, D = q.shape
    scale = D ** -0.5 if scale is None else scale
    out = np.zeros((T, Hq, D))
    t = 0
    for b, (ql, st) in enumerate(zip(q_lens, starts)):
        K = np.asarray(k_seqs[b], dtype=np.float64)
        V = np.asarray(v_seqs[b], dtype=np.float64)
        n_rep = Hq // K.shape[0]
        for i in range(int(ql)):
            p = int(st) + i
            lo, hi = allowed_keys(p, window)
            for h in range(Hq):
                g = h // n_rep
                logits = [sum(q[t + i, h, d] * K[g, j, d] for d in range(D)) * scale for j in range(lo, hi)]
                sink = float(sinks[h])
                m = max(logits + [sink])
                ex = [np.exp(v - m) for v in logits]
                den = sum(ex) + np.exp(sink - m)
                for d in range(D):
                    out[t + i, h, d] = sum(ex[j] * V[g, lo + j, d] for j in range(len(ex))) / den
        t += int(ql)
    return out


def tree_ancestors(par):
    """anc[i] = set of tree nodes on the path root..i, i included (``phase0/tree.py:19-23``)."""
    out = []
    for i in range(len(par)):
        a, j = set(), i
        while j != -1:
            a.add(j)
            j = par[j]
        out.append(a)
    return out


def tree_attention(q, K, V, start, par, dep, sinks, window, scale=None):
    """Tree-verify attention of one sequence (``FastVerify._tset`` masks, ``phase0/fastverify.py:
    250-272``; ``phase0/tree.py:26-46``).  Tree node i is a query at absolute position
    start + dep[i]; its key/value sit at cache slot start + i.  Node i attends

      * every committed prefix key j < start (on sliding layers only if pos_i - j < window);
      * tree slot start + t iff node t is an ancestor of i or i itself (on sliding layers only if
        dep[i] - dep[t] < window).

    q fp32 [M, Hq, D]; K, V fp32 [Hkv, >= start + M, D]; sinks fp32 [Hq].  Softmax with the sink
    column as in ``ragged_attention``.  Returns bf16-valued fp32 [M, Hq, D]."""
    q = torch.as_tensor(q).float()
    M, Hq, D = q.shape
    scale = D ** -0.5 if scale is None else scale
    K = torch.as_tensor(K).float()[:, :start + M]
    V = torch.as_tensor(V).float()[:, :start + M]
    Hkv = K.shape[0]
    n_rep = Hq // Hkv
    anc = tree_ancestors(par)
    allow = torch.zeros(M, start + M, dtype=torch.bool)
    for i in range(M):
        p = start + dep[i]
        for j in range(start):
            allow[i, j] = (not window) or (p - j) < window
        for t in anc[i]:
            allow[i, start + t] = (not window) or (dep[i] - dep[t]) < window
    qq = q.view(M, Hkv, n_rep, D).permute(1, 0, 2, 3)                   # [Hkv, M, n_rep, D]
    s = torch.einsum("gird,gnd->girn", qq, K) * scale
    s = torch.where(allow[None, :, None, :], s, torch.tensor(float("-inf")))
    sk = torch.as_tensor(sinks).float().view(Hkv, 1, n_rep, 1).expand(Hkv, M, n_rep, 1)
    m = torch.maximum(s.amax(dim=-1, keepdim=True), sk)
    e = torch.exp(s - m)
    p = e / (e.sum(dim=-1, keepdim=True) + torch.exp(sk - m))
    o = torch.einsum("girn,gnd->gird", p, V)
    return bf16(o.permute(1, 0, 2, 3).reshape(M, Hq, D))


def brute_force_tree_attention(q, K, V, start, par, dep, sinks, window, scale=None):
    """fp64 pure-Python loops over the reference's dense additive tree mask (``phase0/tree.py:26-46``:
    a finfo.min bias everywhere except the allowed cells); the independent check of the above."""
    q = np.asarray(q, dtype=np.float64)
    K = np.asarray(K, dtype=np.float64)
    V = np.asarray(V, dtype=np.float64)
    M, Hq, D = q.shape
    scale = D ** -0.5 if scale is None else scale
    n_rep = Hq // K.shape[0]
    out = np.zeros((M, Hq, D))
    for i in range(M):
        chain, j = [], i
        while j != -1:
            chain.append(j)
            j = par[j]
        pos_i = start + dep[i]
        keys = [j for j in range(start) if (not window) or pos_i - j < window]
        keys += [start + t for t in range(M) if t in chain and ((not window) or pos_i - (start + dep[t]) < window)]
        for h in range(Hq):
            g = h // n_rep
            logits = [sum(q[i, h, d] * K[g, c, d] for d in range(D)) * scale for c in keys]
            sink = float(sinks[h])
            mx = max(logits + [sink])
            ex = [math.exp(v - mx) for v in logits]
            den = sum(ex) + math.exp(sink - mx)
            for d in range(D):
                out[i, h, d] = sum(ex[c] * V[g, keys[c], d] for c in range(len(keys))) / den
    return out
