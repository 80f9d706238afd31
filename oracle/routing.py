"""Router top-k, expert histogram / stable permute, and unpermute-combine (rows a2, a3, a4).

Numerical contract (shared with the HIP kernels, which must match the INDICES bit-exactly):

* ``dot_fixed`` -- every router logit is an fp32 dot product over K bf16 x bf16 terms in one fixed
  order: 64 lane partials, lane l summing k = 512*j + 8*l + i for j = 0, 1, ... and i = 0..7 (only
  k < K) sequentially (each bf16*bf16 product is exact in fp32, so FMA and mul+add round
  identically), then a xor butterfly over lanes with offsets 32, 16, 8, 4, 2, 1.  Fixing the order
  is what makes the indices reproducible; the lane-contiguous 8-element chunks are what a GPU lane
  reads with one 16-byte load.
* GPT-OSS (``transformers/models/gpt_oss/modeling_gpt_oss.py:126-130``; native MXFP4 path
  ``transformers/integrations/mxfp4.py:476-487``): logits = bf16(dot + bias) -- HF computes the
  router Linear in bf16, so the logits are bf16 values; top-k by (value desc, expert id asc), the
  tie rule of the stable argsort in ``routing_torch_dist`` (``mxfp4.py:435-441``); softmax over
  the k selected values (``mxfp4.py:442``), computed in fp32; each token's k ids are then sorted
  ascending carrying their weights (``mxfp4.py:443-444``).
* DeepSeek-V3 grouped sigmoid (``vendor/kimi_k3_ref/modeling_kimi_linear.py:703-759``): fp32
  logits; scores = sigmoid(logits) via ``sigmoid_det`` (below); selection score = scores + bias;
  group score = sum of the top-2 selection scores in each group; keep ``topk_group`` groups; top-k
  among unmasked experts (ties -> lower id); weights = unbiased scores of the selected experts,
  renormalised by (sum + 1e-20) and multiplied by ``routed_scaling_factor``.  Ids sorted ascending.
* Permute (``mxfp4.py:449-457``; ``modeling_gpt_oss.py:93-107``): hist = bincount; offsets =
  exclusive scan; perm = stable argsort of the flattened [T*k] expert ids (experts ascending, flat
  index t*k+s ascending within an expert); inv = inverse permutation.
* Combine (``modeling_gpt_oss.py:108-113``; ``mxfp4.py:394-403``): fp32 sum over the k slots in
  slot order of weight * y, rounded once to bf16; the residual add (``modeling_gpt_oss.py:375``)
  is bf16(residual + that).

Parity: indices -- brute force (pure-Python loops) and invariants in tests; logits order pinned
by a pure-Python sequential restatement on tiny inputs; weights -- fp64 brute force.
"""
import math

import numpy as np
import torch

from .numerics import bf16


def dot_fixed(x, w):
    """fp32 [T, K] x fp32 [E, K] -> fp32 [T, E] in the fixed 64-lane order described above.
    x and w must hold bf16-representable values (exact products); K % 8 == 0.  Zero padding to a
    multiple of 512 adds exact +0.0 terms to partials that are never -0.0, so it changes nothing."""
    x = torch.as_tensor(x).float()
    w = torch.as_tensor(w).float()
    T, K = x.shape
    E = w.shape[0]
    assert K % 8 == 0, "fixed-order router dot needs K % 8 == 0"
    J = (K + 511) // 512
    pad = J * 512 - K
    if pad:
        x = torch.nn.functional.pad(x, (0, pad))
        w = torch.nn.functional.pad(w, (0, pad))
    xr = x.reshape(T, J, 64, 8)
    wr = w.reshape(E, J, 64, 8)
    out = torch.empty(T, E, dtype=torch.float32)
    idx = torch.arange(64)
    step = max(1, (1 << 24) // max(1, E * 64))          # bound the [t, E, 64] temporaries
    for t0 in range(0, T, step):
        xs = xr[t0:t0 + step]
        acc = torch.zeros(xs.shape[0], E, 64, dtype=torch.float32)
        for j in range(J):
            for i in range(8):
                acc = acc + xs[:, None, j, :, i] * wr[None, :, j, :, i]
        for off in (32, 16, 8, 4, 2, 1):
            acc = acc + acc[..., idx ^ off]
        out[t0:t0 + step] = acc[..., 0]
    return out


def _topk_desc(vals, k):
    """Indices of the k largest values per row, ties -> lower index (stable)."""
    return np.argsort(-vals, axis=1, kind="stable")[:, :k]


def _selection_weights(lg, sel):
    """(ids ascending, fp32 softmax weights in the same order) of a selection sel [T, k] whose rows
    are in (logit desc, id asc) order: the softmax over the k selected logits
    (``transformers/integrations/mxfp4.py:435-447``: top-k, then softmax over the k values)."""
    v = np.take_along_axis(lg, sel, axis=1).astype(np.float32)
    e = np.exp(v - v.max(axis=1, keepdims=True)).astype(np.float32)
    wts = (e / e.sum(axis=1, keepdims=True)).astype(np.float32)
    order = np.argsort(sel, axis=1, kind="stable")
    ids = np.take_along_axis(sel, order, axis=1).astype(np.int32)
    return ids, np.take_along_axis(wts, order, axis=1)


def gptoss_route(x, w, b, k=4):
    """x bf16-valued [T, H], router weight [E, H] and bias [E] (bf16 values).
    Returns (ids int32 [T,k] ascending per row, weights fp32 [T,k], logits fp32 [T,E] bf16-valued)."""
    logits = bf16(dot_fixed(x, w) + torch.as_tensor(b).float()[None, :])
    lg = logits.numpy()
    ids, wts = _selection_weights(lg, _topk_desc(lg, k))
    return ids, wts, logits


def forced_route(logits, ids, wts, force):
    """Teacher forcing, for parity tests: the rows where the expert set ``force`` (int [T, k], e.g. the
    ids a GPU router chose on a near-tie) differs from ``ids`` take force's experts, weighted by the
    same softmax over their logits that gptoss_route applies to its own selection.  Returns
    (ids, weights, the replaced row indices)."""
    lg = np.asarray(logits, dtype=np.float32)
    force = np.sort(np.asarray(force, dtype=np.int64), axis=1)
    rows = np.nonzero((force != np.asarray(ids)).any(axis=1))[0]
    ids, wts = np.array(ids, copy=True), np.array(wts, copy=True)
    if len(rows):
        sub = lg[rows]
        sel = force[rows]
        vals = np.take_along_axis(sub, sel, axis=1)
        sel = np.take_along_axis(sel, np.lexsort((sel, -vals), axis=1), axis=1)  # (logit desc, id asc)
        ids[rows], wts[rows] = _selection_weights(sub, sel)
    return ids, wts, rows


# --- deterministic sigmoid for bit-exact grouped selection -------------------------------------
# exp(z) by Cody-Waite range reduction: n = rint(z * log2 e), r = (z - n*LN2_HI) - n*LN2_LO with
# LN2_HI holding 12 significant bits (so n*LN2_HI is exact), then the degree-7 Taylor polynomial of
# e**r on |r| <= 0.35 by Horner with SEPARATE fp32 multiplies and adds, scaled by 2**n.  sigmoid is
# 1 / (1 + exp(-x)) with a correctly rounded fp32 division.  The HIP kernel performs the same
# operation sequence with __fmul_rn / __fadd_rn / __fdiv_rn, so both sides produce identical bits.
_LOG2E = np.float32(1.4426950408889634)
_LN2_HI = np.float32(0.693145751953125)
_LN2_LO = np.float32(math.log(2.0) - 0.693145751953125)
_P = [np.float32(1.0 / math.factorial(i)) for i in range(8)]


def exp_det(z):
    z = np.clip(np.asarray(z, dtype=np.float32), np.float32(-87.0), np.float32(88.0))
    n = np.rint((z * _LOG2E).astype(np.float32)).astype(np.float32)
    r = (z - (n * _LN2_HI).astype(np.float32)).astype(np.float32)
    r = (r - (n * _LN2_LO).astype(np.float32)).astype(np.float32)
    p = np.full_like(r, _P[7])
    for c in (_P[6], _P[5], _P[4], _P[3], _P[2], _P[1], _P[0]):
        p = (p * r).astype(np.float32)
        p = (p + c).astype(np.float32)
    return np.ldexp(p, n.astype(np.int32)).astype(np.float32)


def sigmoid_det(x):
    x = np.asarray(x, dtype=np.float32)
    e = exp_det(-x)
    return (np.float32(1.0) / (np.float32(1.0) + e).astype(np.float32)).astype(np.float32)


def grouped_sigmoid_route(x, w, e_bias, n_group, topk_group, k, scale):
    """DeepSeek-V3 grouped sigmoid routing (modeling_kimi_linear.py:703-759) on fp32 logits.
    Returns (ids int32 [T,k] ascending, weights fp32 [T,k], scores fp32 [T,E])."""
    logits = dot_fixed(x, w).numpy()
    T, E = logits.shape
    scores = sigmoid_det(logits)
    choice = (scores + np.asarray(e_bias, dtype=np.float32)[None, :]).astype(np.float32)
    if n_group > 1 and n_group > topk_group:
        g = choice.reshape(T, n_group, E // n_group)
        top2 = -np.sort(-g, axis=2)[:, :, :2]
        gscore = (top2[:, :, 0] + top2[:, :, 1]).astype(np.float32)
        gsel = _topk_desc(gscore, topk_group)
        gmask = np.zeros((T, n_group), dtype=bool)
        np.put_along_axis(gmask, gsel, True, axis=1)
        emask = np.repeat(gmask, E // n_group, axis=1)
        masked = np.where(emask, choice, np.float32(-np.inf))
    else:
        masked = choice
    sel = _topk_desc(masked, k)
    order = np.argsort(sel, axis=1, kind="stable")
    ids = np.take_along_axis(sel, order, axis=1).astype(np.int32)
    wsel = np.take_along_axis(scores, ids, axis=1).astype(np.float32)
    # fp32 like the reference (modeling_kimi_linear.py:752-756): sum in ascending id order,
    # (+1e-20), one division, then the scaling factor
    den = np.zeros(T, dtype=np.float32)
    for j in range(k):
        den = (den + wsel[:, j]).astype(np.float32)
    den = (den + np.float32(1e-20)).astype(np.float32)
    wts = ((wsel / den[:, None]).astype(np.float32) * np.float32(scale)).astype(np.float32)
    return ids, wts, scores


def permute(ids, n_experts):
    """ids int [T, k] -> (hist int32[E], offsets int32[E+1], perm int32[T*k], inv int32[T*k])."""
    flat = np.asarray(ids, dtype=np.int64).reshape(-1)
    hist = np.bincount(flat, minlength=n_experts).astype(np.int32)
    offsets = np.zeros(n_experts + 1, dtype=np.int32)
    offsets[1:] = np.cumsum(hist)
    perm = np.argsort(flat, kind="stable").astype(np.int32)
    inv = np.empty_like(perm)
    inv[perm] = np.arange(perm.size, dtype=np.int32)
    return hist, offsets, perm, inv


def combine(y_perm, inv, weights, residual=None):
    """y_perm fp32 [T*k, H] (rows in permuted order), inv [T*k], weights fp32 [T, k].
    Returns bf16-valued fp32 [T, H]: bf16(sum_s w[t,s] * y[inv[t*k+s]]), plus the residual add."""
    y_perm = torch.as_tensor(y_perm).float()
    weights = torch.as_tensor(weights).float()
    T, k = weights.shape
    inv = torch.as_tensor(np.asarray(inv, dtype=np.int64)).view(T, k)
    acc = torch.zeros(T, y_perm.shape[1], dtype=torch.float32)
    for s in range(k):
        acc = acc + weights[:, s, None] * y_perm[inv[:, s]]
    out = bf16(acc)
    if residual is not None:
        out = bf16(torch.as_tensor(residual).float() + out)
    return out
