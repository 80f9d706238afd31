"""Torch-tensor wrappers around the C ABI (one call = one HIP launch sequence on the current stream).

PyTorch provides device memory and the stream; every computation happens in libflyai_stage.so.
Each wrapper checks dtype / device / contiguity / shape on the host before the launch."""
import ctypes as C

import torch

from . import _lib
from ._lib import check, lib


def _stream():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t):
    return C.c_void_p(t.data_ptr()) if t is not None else None


def _need(t, dtype, shape=None, name="tensor"):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be on the GPU")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")
    return t


def pack_ragged(q_lens, starts, kv_base, kv_cap, head_dim, max_tokens):
    """Device int32 q_lens/starts/kv_cap [S], int64 kv_base [S] -> dict of packed index tensors."""
    S = q_lens.numel()
    for n, t, dt in (("q_lens", q_lens, torch.int32), ("starts", starts, torch.int32),
                     ("kv_cap", kv_cap, torch.int32), ("kv_base", kv_base, torch.int64)):
        _need(t, dt, (S,), n)
    dev = q_lens.device
    out = dict(cu_seqlens=torch.empty(S + 1, dtype=torch.int32, device=dev),
               positions=torch.empty(max_tokens, dtype=torch.int32, device=dev),
               seq_id=torch.empty(max_tokens, dtype=torch.int32, device=dev),
               kv_len=torch.empty(S, dtype=torch.int32, device=dev),
               kv_slot=torch.empty(max_tokens, dtype=torch.int64, device=dev),
               status=torch.empty(1, dtype=torch.int32, device=dev))
    check(lib().flyai_pack_ragged(_ptr(q_lens), _ptr(starts), _ptr(kv_base), _ptr(kv_cap), S, head_dim,
                                  max_tokens, _ptr(out["cu_seqlens"]), _ptr(out["positions"]),
                                  _ptr(out["seq_id"]), _ptr(out["kv_len"]), _ptr(out["kv_slot"]),
                                  _ptr(out["status"]), _stream()))
    return out


def router_topk_softmax(x, w, b, k, want_logits=False):
    T, H = x.shape
    E = w.shape[0]
    _need(x, torch.bfloat16, (T, H), "x")
    _need(w, torch.bfloat16, (E, H), "router weight")
    _need(b, torch.bfloat16, (E,), "router bias")
    ids = torch.empty(T, k, dtype=torch.int32, device=x.device)
    wts = torch.empty(T, k, dtype=torch.float32, device=x.device)
    logits = torch.empty(T, E, dtype=torch.float32, device=x.device)
    check(lib().flyai_router_topk_softmax(_ptr(x), _ptr(w), _ptr(b), T, H, E, k, _ptr(ids), _ptr(wts),
                                          _ptr(logits), _stream()))
    return (ids, wts, logits) if want_logits else (ids, wts)


def moe_permute(ids, n_experts):
    T, k = ids.shape
    _need(ids, torch.int32, (T, k), "topk_ids")
    dev = ids.device
    hist = torch.empty(n_experts, dtype=torch.int32, device=dev)
    offsets = torch.empty(n_experts + 1, dtype=torch.int32, device=dev)
    perm = torch.empty(T * k, dtype=torch.int32, device=dev)
    inv = torch.empty(T * k, dtype=torch.int32, device=dev)
    check(lib().flyai_moe_permute(_ptr(ids), T, k, n_experts, _ptr(hist), _ptr(offsets), _ptr(perm),
                                  _ptr(inv), _stream()))
    return hist, offsets, perm, inv


def moe_route_permute(x, w, b, k):
    """Router + histogram/permute as the stage runs it -> (ids, weights, hist, offsets, perm, inv)."""
    T, H = x.shape
    E = w.shape[0]
    _need(x, torch.bfloat16, (T, H), "x")
    _need(w, torch.bfloat16, (E, H), "router weight")
    _need(b, torch.bfloat16, (E,), "router bias")
    dev = x.device
    ids = torch.empty(T, k, dtype=torch.int32, device=dev)
    wts = torch.empty(T, k, dtype=torch.float32, device=dev)
    logits = torch.empty(T, E, dtype=torch.float32, device=dev)
    hist = torch.empty(E, dtype=torch.int32, device=dev)
    offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    perm = torch.empty(T * k, dtype=torch.int32, device=dev)
    inv = torch.empty(T * k, dtype=torch.int32, device=dev)
    check(lib().flyai_moe_route_permute(_ptr(x), _ptr(w), _ptr(b), T, H, E, k, _ptr(ids), _ptr(wts),
                                        _ptr(logits), _ptr(hist), _ptr(offsets), _ptr(perm), _ptr(inv),
                                        _stream()))
    return ids, wts, hist, offsets, perm, inv


def moe_combine(y_perm, inv, topk_w, residual=None, out=None):
    T, k = topk_w.shape
    H = y_perm.shape[1]
    _need(y_perm, torch.float32, (T * k, H), "y_perm")
    _need(inv, torch.int32, (T * k,), "inv")
    _need(topk_w, torch.float32, (T, k), "topk_w")
    if residual is not None:
        _need(residual, torch.bfloat16, (T, H), "residual")
    if out is None:
        out = torch.empty(T, H, dtype=torch.bfloat16, device=y_perm.device)
    _need(out, torch.bfloat16, (T, H), "out")
    check(lib().flyai_moe_combine(_ptr(y_perm), _ptr(inv), _ptr(topk_w), T, k, H, _ptr(residual),
                                  _ptr(out), _stream()))
    return out


def mxfp4_packed_bytes(E, N, K):
    return int(lib().flyai_mxfp4_packed_bytes(E, N, K))


def mxfp4_repack(blocks, scales):
    """HF layout blocks u8 [E, N, K/32, 16] + scales u8 [E, N, K/32] -> packed u8 buffer."""
    E, N, G, _ = blocks.shape
    _need(blocks, torch.uint8, (E, N, G, 16), "blocks")
    _need(scales, torch.uint8, (E, N, G), "scales")
    packed = torch.empty(mxfp4_packed_bytes(E, N, G * 32), dtype=torch.uint8, device=blocks.device)
    check(lib().flyai_mxfp4_repack(_ptr(blocks), _ptr(scales), E, N, G * 32, _ptr(packed), _stream()))
    return packed


def moe_gate_up(x, perm, offsets, k, w13_packed, b13, n_experts, inter):
    T, H = x.shape
    _need(x, torch.bfloat16, (T, H), "x")
    _need(perm, torch.int32, (T * k,), "perm")
    _need(offsets, torch.int32, (n_experts + 1,), "offsets")
    _need(b13, torch.float32, (n_experts, 2 * inter), "b13")
    _need(w13_packed, torch.uint8, (mxfp4_packed_bytes(n_experts, 2 * inter, H),), "w13_packed")
    h = torch.empty(T * k, inter, dtype=torch.bfloat16, device=x.device)
    check(lib().flyai_moe_gate_up_mxfp4(_ptr(x), _ptr(perm), _ptr(offsets), T, k, _ptr(w13_packed),
                                        _ptr(b13), n_experts, H, inter, _ptr(h), _stream()))
    return h


def moe_down(h, offsets, w2_packed, b2, n_experts, hidden):
    P, inter = h.shape
    _need(h, torch.bfloat16, (P, inter), "h")
    _need(offsets, torch.int32, (n_experts + 1,), "offsets")
    _need(b2, torch.float32, (n_experts, hidden), "b2")
    _need(w2_packed, torch.uint8, (mxfp4_packed_bytes(n_experts, hidden, inter),), "w2_packed")
    y = torch.empty(P, hidden, dtype=torch.float32, device=h.device)
    check(lib().flyai_moe_down_mxfp4(_ptr(h), _ptr(offsets), P, _ptr(w2_packed), _ptr(b2), n_experts,
                                     hidden, inter, _ptr(y), _stream()))
    return y


def mx_act_quant(x):
    """bf16 [M, K] -> the two-term e4m3 form: (bytes u8 [2M, K], E8M0 scale bytes u8 [2M, row bytes] in
    MFMA order); row r holds the high term of x[r], row M + r its low term."""
    M, K = x.shape
    _need(x, torch.bfloat16, (M, K), "x")
    q = torch.empty(2 * M, K, dtype=torch.uint8, device=x.device)
    s = torch.empty(int(lib().flyai_mx_act_scale_bytes(2 * M, K)), dtype=torch.uint8, device=x.device)
    check(lib().flyai_mx_act_quant(_ptr(x), M, K, _ptr(q), _ptr(s), _stream()))
    return q, s.view(2 * M, -1) if M else s.view(0, 0)


def moe_gate_up_fp8act(x, xq, xs, perm, offsets, k, w13_packed, b13, n_experts, inter):
    """gate_up with the dense groups on the scaled MFMA (two-term fp8 activations xq/xs = mx_act_quant(x))."""
    T, H = x.shape
    _need(x, torch.bfloat16, (T, H), "x")
    _need(xq, torch.uint8, (2 * T, H), "xq")
    _need(xs, torch.uint8, (2 * T, int(lib().flyai_mx_act_scale_bytes(1, H))), "xs")
    _need(perm, torch.int32, (T * k,), "perm")
    _need(offsets, torch.int32, (n_experts + 1,), "offsets")
    _need(b13, torch.float32, (n_experts, 2 * inter), "b13")
    _need(w13_packed, torch.uint8, (mxfp4_packed_bytes(n_experts, 2 * inter, H),), "w13_packed")
    h = torch.empty(T * k, inter, dtype=torch.bfloat16, device=x.device)
    check(lib().flyai_moe_gate_up_mxfp4_fp8act(_ptr(x), _ptr(xq), _ptr(xs), _ptr(perm), _ptr(offsets), T, k,
                                               _ptr(w13_packed), _ptr(b13), n_experts, H, inter, _ptr(h),
                                               _stream()))
    return h


def moe_down_fp8act(h, hq, hs, offsets, w2_packed, b2, n_experts, hidden):
    """down with the dense groups on the scaled MFMA (two-term fp8 activations hq/hs = mx_act_quant(h))."""
    P, I = h.shape
    _need(h, torch.bfloat16, (P, I), "h")
    _need(hq, torch.uint8, (2 * P, I), "hq")
    _need(hs, torch.uint8, (2 * P, int(lib().flyai_mx_act_scale_bytes(1, I))), "hs")
    _need(offsets, torch.int32, (n_experts + 1,), "offsets")
    _need(b2, torch.float32, (n_experts, hidden), "b2")
    _need(w2_packed, torch.uint8, (mxfp4_packed_bytes(n_experts, hidden, I),), "w2_packed")
    y = torch.empty(P, hidden, dtype=torch.float32, device=h.device)
    check(lib().flyai_moe_down_mxfp4_fp8act(_ptr(h), _ptr(hq), _ptr(hs), _ptr(offsets), P, _ptr(w2_packed),
                                            _ptr(b2), n_experts, hidden, I, _ptr(y), _stream()))
    return y


def rmsnorm(x, w, eps=1e-5):
    T, H = x.shape
    _need(x, torch.bfloat16, (T, H), "x")
    _need(w, torch.float32, (H,), "weight")
    y = torch.empty_like(x)
    check(lib().flyai_rmsnorm(_ptr(x), _ptr(w), T, H, eps, _ptr(y), _stream()))
    return y


def linear(x, w, b=None, residual=None):
    """y = bf16(x W^T + b); with residual, residual <- bf16(residual + y) (returned)."""
    M, K = x.shape
    N = w.shape[0]
    _need(x, torch.bfloat16, (M, K), "x")
    _need(w, torch.bfloat16, (N, K), "weight")
    if b is not None:
        _need(b, torch.bfloat16, (N,), "bias")
    y = None
    if residual is not None:
        _need(residual, torch.bfloat16, (M, N), "residual")
    else:
        y = torch.empty(M, N, dtype=torch.bfloat16, device=x.device)
    ws = torch.empty(max(1, int(lib().flyai_linear_workspace_bytes(M, N, K)) // 4), dtype=torch.float32,
                     device=x.device)
    check(lib().flyai_linear_bf16(_ptr(x), _ptr(w), _ptr(b), M, N, K, _ptr(y), _ptr(residual), _ptr(ws),
                                  _stream()))
    return residual if residual is not None else y


def rope_kv_append(qkv, positions, seq_id, cos_tab, sin_tab, n_q_heads, n_kv_heads, head_dim,
                   kv_base, kv_cap, k_pool, v_pool):
    T = qkv.shape[0]
    _need(qkv, torch.bfloat16, (T, (n_q_heads + 2 * n_kv_heads) * head_dim), "qkv")
    _need(positions, torch.int32, None, "positions")
    _need(seq_id, torch.int32, None, "seq_id")
    _need(cos_tab, torch.bfloat16, None, "cos")
    _need(sin_tab, torch.bfloat16, cos_tab.shape, "sin")
    _need(kv_base, torch.int64, None, "kv_base")
    _need(kv_cap, torch.int32, kv_base.shape, "kv_cap")
    _need(k_pool, torch.bfloat16, None, "k_pool")
    _need(v_pool, torch.bfloat16, k_pool.shape, "v_pool")
    if positions.numel() < T or seq_id.numel() < T:
        raise ValueError("positions/seq_id shorter than the token count")
    q = torch.empty(T, n_q_heads, head_dim, dtype=torch.bfloat16, device=qkv.device)
    check(lib().flyai_rope_kv_append(_ptr(qkv), _ptr(positions), _ptr(seq_id), _ptr(cos_tab),
                                     _ptr(sin_tab), cos_tab.shape[0], T, n_q_heads, n_kv_heads, head_dim, _ptr(kv_base),
                                     _ptr(kv_cap), _ptr(q), _ptr(k_pool), _ptr(v_pool), _stream()))
    return q


def attn_plan(q_lens, starts, n_kv_heads, window, split_keys, max_items=1 << 20):
    """Host planner -> (items int32 [n, 8], groups int32 [g, 8], n_small) on the CPU."""
    S = len(q_lens)
    ql = (C.c_int32 * S)(*[int(v) for v in q_lens])
    st = (C.c_int32 * S)(*[int(v) for v in starts])
    max_groups = (S + sum((int(v) + 3) // 4 for v in q_lens)) * n_kv_heads
    items = (_lib.AttnItem * max_items)()
    groups = (_lib.AttnGroup * max_groups)()
    ni, ng, ns = C.c_int32(0), C.c_int32(0), C.c_int32(0)
    check(lib().flyai_attn_plan(ql, st, S, n_kv_heads, window, split_keys, items, max_items, groups,
                                max_groups, C.byref(ni), C.byref(ng), C.byref(ns)))
    it = torch.frombuffer(bytearray(items), dtype=torch.int32).view(max_items, 8)[:ni.value].clone()
    gr = torch.frombuffer(bytearray(groups), dtype=torch.int32).view(max_groups, 8)[:ng.value].clone()
    return it, gr, ns.value


def attn_plan_prefill(q_lens, starts, n_kv_heads, window, split_keys, prefill_min, max_items=1 << 20):
    """attn_plan with sequences of q_len >= prefill_min as prefill items -> (items, groups, n_small,
    pitems) on the CPU."""
    S = len(q_lens)
    ql = (C.c_int32 * S)(*[int(v) for v in q_lens])
    st = (C.c_int32 * S)(*[int(v) for v in starts])
    max_groups = (S + sum((int(v) + 3) // 4 for v in q_lens)) * n_kv_heads
    max_pitems = (S + sum((int(v) + 15) // 16 for v in q_lens)) * n_kv_heads
    items = (_lib.AttnItem * max_items)()
    groups = (_lib.AttnGroup * max_groups)()
    pitems = (_lib.AttnItem * max_pitems)()
    ni, ng, ns, npi = C.c_int32(0), C.c_int32(0), C.c_int32(0), C.c_int32(0)
    check(lib().flyai_attn_plan_prefill(ql, st, S, n_kv_heads, window, split_keys, prefill_min, items, max_items,
                                        groups, max_groups, pitems, max_pitems, C.byref(ni), C.byref(ng),
                                        C.byref(ns), C.byref(npi)))
    it = torch.frombuffer(bytearray(items), dtype=torch.int32).view(max_items, 8)[:ni.value].clone()
    gr = torch.frombuffer(bytearray(groups), dtype=torch.int32).view(max_groups, 8)[:ng.value].clone()
    pit = torch.frombuffer(bytearray(pitems), dtype=torch.int32).view(max_pitems, 8)[:npi.value].clone()
    return it, gr, ns.value, pit


def attn_prefill(q, k_pool, v_pool, kv_base, kv_cap, sinks, window, pitems, n_kv_heads, out):
    """Run prefill items (attn_plan_prefill) into the rows of out bf16 [T, Hq, 64]."""
    T, Hq, D = q.shape
    _need(q, torch.bfloat16, (T, Hq, D), "q")
    _need(out, torch.bfloat16, (T, Hq, D), "out")
    pit = pitems.to(q.device).contiguous()
    check(lib().flyai_attn_prefill(_ptr(q), _ptr(k_pool), _ptr(v_pool), _ptr(kv_base), _ptr(kv_cap), _ptr(sinks),
                                   window, Hq, n_kv_heads, D, _ptr(pit), pitems.shape[0], _ptr(out), _stream()))
    return out


def attn_ragged(q, k_pool, v_pool, kv_base, kv_cap, sinks, window, items, groups, n_small, n_kv_heads):
    """q bf16 [T, Hq, 64]; items/groups/n_small from attn_plan (moved to the GPU here)."""
    T, Hq, D = q.shape
    _need(q, torch.bfloat16, (T, Hq, D), "q")
    _need(sinks, torch.float32, (Hq,), "sinks")
    dev = q.device
    items_d = items.to(dev).contiguous()
    groups_d = groups.to(dev).contiguous()
    parts = torch.empty(max(1, int(lib().flyai_attn_partials_bytes(items.shape[0])) // 4),
                        dtype=torch.float32, device=dev)
    out = torch.empty_like(q)
    check(lib().flyai_attn_ragged(_ptr(q), _ptr(k_pool), _ptr(v_pool), _ptr(kv_base), _ptr(kv_cap),
                                  _ptr(sinks), window, Hq, n_kv_heads, D, _ptr(items_d), items.shape[0],
                                  n_small, _ptr(groups_d), groups.shape[0], _ptr(parts), _ptr(out),
                                  _stream()))
    return out


# ---- DeepSeek-V3-shaped FP8 MoE ------------------------------------------------------------------

def router_grouped_sigmoid(x, w, e_bias, n_group, topk_group, k, route_scale):
    """Grouped sigmoid routing on fp32 logits -> (ids int32 [T,k] ascending, weights fp32 [T,k],
    logits fp32 [T,E])."""
    T, H = x.shape
    E = w.shape[0]
    _need(x, torch.bfloat16, (T, H), "x")
    _need(w, torch.bfloat16, (E, H), "router weight")
    if e_bias is not None:
        _need(e_bias, torch.float32, (E,), "e_bias")
    dev = x.device
    logits = torch.empty(T, E, dtype=torch.float32, device=dev)
    ids = torch.empty(T, k, dtype=torch.int32, device=dev)
    wts = torch.empty(T, k, dtype=torch.float32, device=dev)
    check(lib().flyai_router_grouped_sigmoid(_ptr(x), _ptr(w), _ptr(e_bias), T, H, E, n_group, topk_group,
                                             k, float(route_scale), _ptr(logits), _ptr(ids), _ptr(wts),
                                             _stream()))
    return ids, wts, logits


def fp8_act_quant(x):
    """bf16 [M, K] -> (e4m3 bytes u8 [M, K], E8M0 scale bytes u8 [M, K/128])."""
    M, K = x.shape
    _need(x, torch.bfloat16, (M, K), "x")
    q = torch.empty(M, K, dtype=torch.uint8, device=x.device)
    s = torch.empty(M, K // 128, dtype=torch.uint8, device=x.device)
    check(lib().flyai_fp8_act_quant(_ptr(x), M, K, _ptr(q), _ptr(s), _stream()))
    return q, s


def fp8_packed_bytes(E, N, K):
    return int(lib().flyai_fp8_packed_bytes(E, N, K))


def fp8_repack(w1, s1, w3=None, s3=None):
    """e4m3 bytes w [E, N, K] + E8M0 block scales [E, ceil(N/128), K/128] -> packed u8 buffer.
    With w3/s3 (gate_up), rows of w1 and w3 are interleaved and the packed N is 2N."""
    E, N, K = w1.shape
    sb = (E, (N + 127) // 128, K // 128)
    _need(w1, torch.uint8, (E, N, K), "w1")
    _need(s1, torch.uint8, sb, "s1")
    if w3 is not None:
        _need(w3, torch.uint8, (E, N, K), "w3")
        _need(s3, torch.uint8, sb, "s3")
    Np = 2 * N if w3 is not None else N
    packed = torch.empty(fp8_packed_bytes(E, Np, K), dtype=torch.uint8, device=w1.device)
    check(lib().flyai_fp8_repack(_ptr(w1), _ptr(s1), _ptr(w3), _ptr(s3), E, N, K, _ptr(packed), _stream()))
    return packed


def moe_gate_up_fp8(xq, xs, perm, offsets, k, topk_w, w13_packed, n_experts, inter, n_shared=0):
    """Rows of expert e: token perm[p] // k (perm None: token p); h = bf16(silu(bf16 gate) * bf16 up
    * topk_w[perm[p]]) (topk_w None: 1) -> h bf16 [P + n_shared, inter], P = routed rows.  With
    n_shared > 0 the packed buffer holds the shared expert as expert n_experts; its rows P.. take
    tokens 0 .. n_shared-1 with weight 1."""
    T, H = xq.shape
    _need(xq, torch.uint8, (T, H), "xq")
    _need(xs, torch.uint8, (T, H // 128), "xs")
    _need(offsets, torch.int32, (n_experts + 1,), "offsets")
    if not 0 <= n_shared <= T:
        raise ValueError("n_shared must be in [0, T]")
    P = T * k if perm is not None else T
    if perm is not None:
        _need(perm, torch.int32, (P,), "perm")
    if topk_w is not None:
        _need(topk_w, torch.float32, None, "topk_w")
        if topk_w.numel() != P:
            raise ValueError("topk_w must hold one weight per routed row")
    groups = n_experts + (n_shared > 0)
    _need(w13_packed, torch.uint8, (fp8_packed_bytes(groups, 2 * inter, H),), "w13_packed")
    h = torch.empty(P + n_shared, inter, dtype=torch.bfloat16, device=xq.device)
    check(lib().flyai_moe_gate_up_fp8(_ptr(xq), _ptr(xs), _ptr(perm), _ptr(offsets), k, _ptr(topk_w),
                                      _ptr(w13_packed), n_experts, H, inter, n_shared, _ptr(h), _stream()))
    return h


def moe_down_fp8(hq, hs, offsets, w2_packed, n_experts, hidden, n_shared=0):
    """y[p] = bf16(hq[p] . W2[e]) for routed rows and, with n_shared > 0, the shared expert's rows
    (the last n_shared rows of hq) -> y bf16 [rows, hidden]."""
    R, inter = hq.shape
    _need(hq, torch.uint8, (R, inter), "hq")
    _need(hs, torch.uint8, (R, inter // 128), "hs")
    _need(offsets, torch.int32, (n_experts + 1,), "offsets")
    groups = n_experts + (n_shared > 0)
    _need(w2_packed, torch.uint8, (fp8_packed_bytes(groups, hidden, inter),), "w2_packed")
    y = torch.empty(R, hidden, dtype=torch.bfloat16, device=hq.device)
    check(lib().flyai_moe_down_fp8(_ptr(hq), _ptr(hs), _ptr(offsets), _ptr(w2_packed), n_experts, hidden,
                                   inter, n_shared, _ptr(y), _stream()))
    return y


def moe_combine_sum(y_perm, inv, k, shared=None, residual=None, out=None):
    """out[t] = bf16(sum_s y_perm[inv[t*k+s]] + shared[t]) (fp32), then bf16(residual + out)."""
    P, H = y_perm.shape
    T = P // k
    _need(y_perm, torch.bfloat16, (P, H), "y_perm")
    _need(inv, torch.int32, (P,), "inv")
    for n, t in (("shared", shared), ("residual", residual)):
        if t is not None:
            _need(t, torch.bfloat16, (T, H), n)
    if out is None:
        out = torch.empty(T, H, dtype=torch.bfloat16, device=y_perm.device)
    _need(out, torch.bfloat16, (T, H), "out")
    check(lib().flyai_moe_combine_sum(_ptr(y_perm), _ptr(inv), T, k, H, _ptr(shared), _ptr(residual),
                                      _ptr(out), _stream()))
    return out


def bf16_tile_repack(w):
    """nn.Linear weight bf16 [N, K] -> MFMA-fragment tiles (u8 buffer) for lm_head_argmax."""
    N, K = w.shape
    _need(w, torch.bfloat16, (N, K), "w")
    n = int(lib().flyai_bf16_tile_packed_bytes(N, K))
    if n == 0:
        raise ValueError("bf16_tile_repack needs N % 16 == 0 and K % 32 == 0")
    packed = torch.empty(n, dtype=torch.uint8, device=w.device)
    check(lib().flyai_bf16_tile_repack(_ptr(w), N, K, _ptr(packed), _stream()))
    return packed


def embed_gather(table, ids):
    """table bf16 [V, H], ids int32 [T] (device) -> bf16 [T, H]."""
    V, H = table.shape
    _need(table, torch.bfloat16, (V, H), "table")
    _need(ids, torch.int32, None, "ids")
    out = torch.empty(ids.numel(), H, dtype=torch.bfloat16, device=table.device)
    check(lib().flyai_embed_gather(_ptr(table), _ptr(ids), ids.numel(), H, V, _ptr(out), _stream()))
    return out


def lm_head_argmax(x, w_packed, vocab, rows=None, want_logits=False, workspace=None):
    """Greedy token of each selected row: x bf16 [R, H] final-normed hidden rows; rows int32 [n]
    (device; None: all R rows); returns ids int32 [n] (and bf16 logits [n, vocab])."""
    R, H = x.shape
    _need(x, torch.bfloat16, (R, H), "x")
    n = R if rows is None else rows.numel()
    if rows is not None:
        _need(rows, torch.int32, (n,), "rows")
    _need(w_packed, torch.uint8, (int(lib().flyai_bf16_tile_packed_bytes(vocab, H)),), "w_packed")
    ids = torch.empty(n, dtype=torch.int32, device=x.device)
    logits = torch.empty(n, vocab, dtype=torch.bfloat16, device=x.device) if want_logits else None
    need = int(lib().flyai_lm_head_workspace_bytes(n, vocab))
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=x.device)
    check(lib().flyai_lm_head_argmax(_ptr(x), _ptr(rows), n, H, _ptr(w_packed), vocab, _ptr(ids),
                                     _ptr(logits), _ptr(workspace), _stream()))
    return (ids, logits) if want_logits else ids


def sample_rows(logits, temp, top_k=0, top_p=1.0, draft=None, u=None, want_p_draft=False, want_draw=False,
                want_probs=False):
    """Temperature / top-k / top-p over bf16 logits rows [R, V] (one workgroup per row).  draft int32 [R]
    (device, -1 = none) and u float64 [R] (device uniforms in [0, 1)) are optional; returns a dict with
    the requested outputs: p_draft fp32 [R], draw int32 [R] (needs u unless temp <= 0), probs fp32 [R, V]."""
    R, V = logits.shape
    _need(logits, torch.bfloat16, (R, V), "logits")
    if draft is not None:
        _need(draft, torch.int32, (R,), "draft")
    if u is not None:
        _need(u, torch.float64, (R,), "u")
    if want_draw and u is None and temp > 0:
        raise ValueError("a sampled draw needs uniforms u")
    dev = logits.device
    out = {}
    if want_p_draft:
        out["p_draft"] = torch.empty(R, dtype=torch.float32, device=dev)
    if want_draw:
        out["draw"] = torch.empty(R, dtype=torch.int32, device=dev)
    if want_probs:
        out["probs"] = torch.empty(R, V, dtype=torch.float32, device=dev)
    check(lib().flyai_sample_rows(_ptr(logits), R, V, float(temp), int(top_k), float(top_p), _ptr(draft), _ptr(u),
                                  _ptr(out.get("p_draft")), _ptr(out.get("draw")), _ptr(out.get("probs")),
                                  _stream()))
    return out


def sample_probs(probs, u):
    """One draw from a fp32 probability vector [V] (device) at uniform u in [0, 1): int32 [1] on device."""
    V = probs.numel()
    _need(probs, torch.float32, (V,), "probs")
    out = torch.empty(1, dtype=torch.int32, device=probs.device)
    check(lib().flyai_sample_probs(_ptr(probs), V, float(u), _ptr(out), _stream()))
    return out
