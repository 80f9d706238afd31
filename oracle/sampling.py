"""Token sampling: temperature, top-k, top-p, the speculative-sampling accept rule (row f1).

Follows the tail's ``Sampler`` (``phase0/specsample.py:36-107``):

    dist(x)   z = fp32(x) / max(temp, 1e-6)                                       (:55)
              top-k: keep z >= the k-th largest z (0 < k < V)                       (:56-58)
              p = softmax(z); top-p (0 < top_p < 1): sort p descending, keep a token
              while (cumsum - p) <= top_p, renormalise                              (:59-66)
    accept    slot j: accept d_j iff u < p_j(d_j); on the first rejection draw from
              p_j with d_j removed (argmax of p_j when nothing is left); when all K
              accept, one bonus draw from p_K                                      (:79-107)
    greedy    temp <= 0: argmax of the logits row                                   (:75-77, :89-90)

Restated over exact integer weights so that the GPU kernel can match it bit for bit whatever its
reduction order: w_v = floor(2^40 e^(z_v - max z)) with e^d computed by ``samp_exp`` (fixed fp64
operations, the same ones the kernel issues), top-p compares integer prefix sums against
floor(top_p * W), and a draw with uniform u is the inverse CDF at floor(u * W) over the weights in id
order.  Ties in the sorted order are broken by ascending id (-0 and +0 are one value); the reference's
``torch.sort`` leaves that order unspecified.

The random numbers are the caller's: the reference's torch generator and multinomial cannot be
reproduced, so parity of a draw is pinned for given uniforms, and the distribution of the whole
accept protocol is pinned by its losslessness (every slot's output is distributed as p).

Parity: ``samp_exp`` against math.exp within one weight unit over its whole range; ``dist`` against
the literal fp64 float-probability formula of the reference (tests/test_oracle_sampling.py);
greedy against numpy argmax; hand-computed known answers; Monte-Carlo losslessness of ``accept``.
"""
import math

import numpy as np

ONE = 1 << 40                              # weight of the most likely token
_INV_LN2 = float.fromhex("0x1.71547652b82fep+0")
_LN2_HI = float.fromhex("0x1.62e42feep-1")  # 32 significant bits: k * _LN2_HI is exact for |k| <= 40
_LN2_LO = float.fromhex("0x1.a39ef35793c76p-33")
_TAYLOR = [1.0 / math.factorial(n) for n in range(14)]   # e^r = sum r^n / n!, n <= 13
_CUTOFF = -27.75                           # 2^40 e^d < 1 below this


def samp_exp(d):
    """floor(2^40 e^d) for fp64 d <= 0 (array), as uint64: Cody-Waite reduction d = k ln2 + r with ln2
    split into a 32-bit head and a tail, then the degree-13 Taylor polynomial of e^r by Horner, every
    operation one rounded fp64 multiply or add (numpy fuses nothing)."""
    d = np.asarray(d, dtype=np.float64)
    live = d >= _CUTOFF
    d = np.where(live, d, 0.0)
    k = np.rint(d * _INV_LN2)
    r = (d - k * _LN2_HI) - k * _LN2_LO
    p = np.full_like(d, _TAYLOR[13])
    for n in range(12, -1, -1):
        p = p * r + _TAYLOR[n]
    e = k.astype(np.int64) + 40
    w = np.floor(np.ldexp(p, e))
    return np.where(live, w, 0.0).astype(np.uint64)


def _canon(z):
    z = np.asarray(z, dtype=np.float32).copy()
    z[z == 0] = 0.0                        # -0 -> +0
    return z


def _desc_order(z):
    """Indices of z sorted by (value desc, id asc)."""
    ids = np.arange(z.size)
    return np.lexsort((ids, -z.astype(np.float64)))


def weights(x, temp, top_k=0, top_p=1.0):
    """Kept integer weights of one logits row x (float32 values of the bf16 logits): uint64 [V]."""
    x = np.asarray(x, dtype=np.float32)
    V = x.size
    z = _canon(x / np.float32(max(np.float32(temp), np.float32(1e-6))))
    keep = np.ones(V, dtype=bool)
    if 0 < top_k < V:
        kth = np.sort(z)[V - top_k]                     # k-th largest, counted with multiplicity
        keep = z >= kth
    zmax = z.max()
    w = samp_exp(z.astype(np.float64) - np.float64(zmax))
    w[~keep] = 0
    top_p = float(np.float32(top_p))
    if 0.0 < top_p < 1.0:
        W = int(w.sum(dtype=np.uint64))
        T = math.floor(top_p * float(W))
        order = _desc_order(np.where(keep, z, -np.inf).astype(np.float32))
        ws = w[order]
        before = np.cumsum(ws, dtype=np.uint64) - ws
        ws[before > np.uint64(T)] = 0
        w = np.zeros_like(w)
        w[order] = ws
    return w


def probs(w):
    """fp32 probabilities of integer weights (one fp64 division each)."""
    W = float(int(w.sum(dtype=np.uint64)))
    return (w.astype(np.float64) / W).astype(np.float32)


def p_of(w, v):
    """fp32 probability of token v under weights w."""
    return np.float32(float(int(w[v])) / float(int(w.sum(dtype=np.uint64))))


def draw(w, u, exclude=-1):
    """Inverse-CDF draw at uniform u over w in id order, token ``exclude`` removed (the residual);
    when nothing is left, the first id of maximal w."""
    r = w.copy()
    if exclude >= 0:
        r[exclude] = 0
    cum = np.cumsum(r, dtype=np.uint64)
    Wr = int(cum[-1])
    if Wr == 0:
        return int(np.argmax(w))
    target = min(int(u * float(Wr)), Wr - 1)
    return int(np.searchsorted(cum, np.uint64(target), side="right"))


def draw_probs(p, u):
    """A draw from a probability vector (Sampler.sample): weights floor(p * 2^40), then ``draw``;
    0 when every weight is 0."""
    w = np.floor(np.maximum(np.asarray(p, dtype=np.float32), 0).astype(np.float64) * ONE).astype(np.uint64)
    if int(w.sum(dtype=np.uint64)) == 0:
        return 0
    return draw(w, u)


def greedy(x):
    """argmax of a logits row, first occurrence."""
    return int(np.argmax(_canon(x)))


def accept(logits, draft, temp, top_k, top_p, uniforms):
    """The speculative-sampling result list r (length K+1) for a deterministic draft, consuming
    ``uniforms`` (an iterator of floats in [0, 1)) in the kernel-backed Sampler's order: one per
    examined slot, then one for the residual or bonus draw."""
    K = len(draft)
    if temp <= 0:
        return [greedy(row) for row in logits]
    r = [0] * (K + 1)
    for j in range(K):
        w = weights(logits[j], temp, top_k, top_p)
        if next(uniforms) < float(p_of(w, draft[j])):
            r[j] = draft[j]
            continue
        r[j] = draw(w, next(uniforms), exclude=draft[j])
        return r
    r[K] = draw(weights(logits[K], temp, top_k, top_p), next(uniforms))
    return r
