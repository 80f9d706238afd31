"""Stage runtimes over libflyai_stage: a ragged continuous-batch step, plus classes that keep the
call surface of the reference's stage runtimes so they drop in for that path.

* ``RaggedStage.forward(hidden, q_lens, starts, slots)`` -- one step over a flat token batch that
  mixes decode rows (q=1), spec-verify rows (q=K+1) and chunked-prefill rows (q=chunk).
* ``FastVerifyStage`` -- ``FastVerify`` (phase0/fastverify.py:80-309): ``reset``, ``prefill(h, start)``,
  ``decode(h, start)``, ``tree_decode`` (ancestor-masked tree verify), ``tree_gather``; raises
  ``ContextOverflow`` before any write.
* ``BatchedFastVerifyStage`` -- ``BatchedFastVerify`` (phase0/batchverify.py:64-190): ``reset``,
  ``load_prefix(b, src)``, ``decode(h[B, kp1, H], starts[B], use_graph=True)``.

The KV workspace is one slab per sequence slot in per-layer pools, each kv head a region of cap x 64
tiled in 64-key blocks in the attention kernel's fragment order (flyai_amd.kvlayout).  It replaces
StaticKV / BatchedStaticKV ([B, Hkv, maxlen, D] per layer, fastverify.py:52-77,
batchverify.py:29-48)."""
import ctypes as C

import numpy as np
import torch

from . import _lib, kvlayout, ops, stage_parts
from ._lib import ContextOverflow, check, lib
from .weights import GptOssShape


def _round_up(v, m):
    return (v + m - 1) // m * m


class KVWorkspace:
    """Per-layer K/V pools holding ``n_slots`` sequence slabs in the tiled layout of
    ``flyai_amd.kvlayout`` (what the attention kernel streams).  Every slab holds ``maxlen`` positions,
    or slot i holds ``caps[i]`` (a per-sequence workspace sized to each sequence's context); a slab's
    capacity is rounded up to a multiple of 64 positions."""

    def __init__(self, n_layers, n_slots, maxlen, n_kv_heads=8, head_dim=64, device="cuda", caps=None):
        if head_dim != kvlayout.HEAD_DIM:
            raise ValueError("the tiled KV layout needs head_dim 64")
        if caps is None:
            caps = [maxlen] * n_slots
        if len(caps) != n_slots or min(caps) < 1:
            raise ValueError("caps needs one positive capacity per slot")
        self.n_layers, self.n_slots = n_layers, n_slots
        self.maxlens = [int(c) for c in caps]
        self.caps = [_round_up(max(int(c), 64), 64) for c in caps]
        self.maxlen = max(self.maxlens)
        self.cap = max(self.caps)
        self.n_kv_heads, self.head_dim = n_kv_heads, head_dim
        self.slabs = [n_kv_heads * c * head_dim for c in self.caps]
        self.bases = np.concatenate([[0], np.cumsum(self.slabs)]).astype(np.int64)
        self.slab = self.slabs[0]
        n = int(self.bases[-1])
        self.k = [torch.zeros(n, dtype=torch.bfloat16, device=device) for _ in range(n_layers)]
        self.v = [torch.zeros(n, dtype=torch.bfloat16, device=device) for _ in range(n_layers)]

    def base(self, slot):
        return int(self.bases[slot])

    def slot_cap(self, slot):
        return self.caps[slot]

    def zero(self):
        for t in self.k + self.v:
            t.zero_()

    def _slab(self, pools, layer, slot):
        return pools[layer][self.base(slot):self.base(slot) + self.slabs[slot]]

    def k_dense(self, layer, slot, positions=None):
        """Dense [Hkv, P, 64] copy of one slot's keys (all cap positions by default)."""
        return kvlayout.gather(self._slab(self.k, layer, slot), self.n_kv_heads, self.caps[slot], "k", positions)

    def v_dense(self, layer, slot, positions=None):
        """Dense [Hkv, P, 64] copy of one slot's values."""
        return kvlayout.gather(self._slab(self.v, layer, slot), self.n_kv_heads, self.caps[slot], "v", positions)

    def set_dense(self, layer, slot, k, v, positions=None):
        """Write dense [Hkv, P, 64] keys and values into one slot."""
        kvlayout.scatter(self._slab(self.k, layer, slot), self.n_kv_heads, self.caps[slot], "k", k, positions)
        kvlayout.scatter(self._slab(self.v, layer, slot), self.n_kv_heads, self.caps[slot], "v", v, positions)

    def move_positions(self, layer, slot, src, dst):
        """K/V rows at positions src -> positions dst (all read before any is written)."""
        k, v = self.k_dense(layer, slot, src), self.v_dense(layer, slot, src)
        self.set_dense(layer, slot, k, v, dst)

    def copy_slot(self, dst, src_ws, src_slot=0):
        if src_ws.caps[src_slot] != self.caps[dst] or src_ws.n_kv_heads != self.n_kv_heads:
            raise ValueError("load_prefix needs workspaces of the same capacity and heads")
        for l in range(self.n_layers):
            self._slab(self.k, l, dst).copy_(src_ws._slab(src_ws.k, l, src_slot))
            self._slab(self.v, l, dst).copy_(src_ws._slab(src_ws.v, l, src_slot))


class RaggedStage:
    """One pipeline stage of GPT-OSS decoder layers on libflyai_stage."""

    def __init__(self, shape: GptOssShape, layers, rotary, kv: KVWorkspace, max_tokens, max_seqs,
                 max_attn_items=None, split_keys=1024, device="cuda", use_graphs=False, prefill_min=32,
                 dense_fp8=False):
        """dense_fp8: expert groups large enough for the dense kernels run on the scaled f8f6f4 MFMA with
        two-term fp8 activation operands (within fp32 accumulation order of the bf16 path, slower on
        groups of a 2048-token prefill chunk); the default keeps them on bf16 activations, bit-identical to the decode path."""
        self.shape, self.layers, self.rotary, self.kv = shape, layers, rotary, kv
        self.device = torch.device(device)
        self.max_tokens, self.max_seqs = max_tokens, max_seqs
        if max_attn_items is None:
            groups = (max_seqs + (max_tokens + 3) // 4) * shape.n_kv_heads
            max_attn_items = groups * max(1, -(-kv.cap // split_keys))
        cfg = _lib.StageConfig(
            n_layers=len(layers), hidden=shape.hidden, n_q_heads=shape.n_q_heads,
            n_kv_heads=shape.n_kv_heads, head_dim=shape.head_dim, n_experts=shape.n_experts,
            top_k=shape.top_k, intermediate=shape.intermediate, window=shape.window,
            max_tokens=max_tokens, max_seqs=max_seqs, max_attn_items=max_attn_items,
            rope_positions=rotary.n_positions, attn_split_keys=split_keys, rms_eps=shape.rms_eps,
            attn_prefill_min=prefill_min, moe_dense_fp8=int(bool(dense_fp8)))
        self.dense_fp8 = bool(dense_fp8)
        handle = C.c_void_p()
        check(lib().flyai_stage_create(C.byref(cfg), C.byref(handle)))
        self._h = handle
        # held here: at interpreter exit the module globals the destructor would reach may be gone
        self._destroy = lib().flyai_stage_destroy
        self._sync = torch.cuda.synchronize
        self.layers = list(layers)
        for i, lw in enumerate(layers):
            self.set_layer(i, lw)
        check(lib().flyai_stage_set_rope(self._h, C.c_void_p(rotary.cos.data_ptr()),
                                         C.c_void_p(rotary.sin.data_ptr())))
        host_bytes = int(lib().flyai_stage_host_staging_bytes(self._h))
        self.staging = torch.empty(host_bytes, dtype=torch.uint8, pin_memory=True)
        self.set_workspace()
        self.use_graphs = False
        self.set_graphs(use_graphs)

    def set_layer(self, i, lw):
        """Bind layer i to the weights of ``lw`` and the workspace's layer-i KV pools.  Drops every
        captured step graph (they hold the previous pointers)."""
        kv = self.kv
        d = _lib.LayerDesc(
            ln1=lw.ln1.data_ptr(), ln2=lw.ln2.data_ptr(), wqkv=lw.wqkv.data_ptr(),
            bqkv=lw.bqkv.data_ptr(), wo=lw.wo.data_ptr(), bo=lw.bo.data_ptr(),
            sinks=lw.sinks.data_ptr(), router_w=lw.router_w.data_ptr(),
            router_b=lw.router_b.data_ptr(), w13_packed=lw.w13_packed.data_ptr(),
            b13=lw.b13.data_ptr(), w2_packed=lw.w2_packed.data_ptr(), b2=lw.b2.data_ptr(),
            k_pool=kv.k[i].data_ptr(), v_pool=kv.v[i].data_ptr(), sliding=int(lw.sliding), pad=0,
            kv_pool_elems=min(kv.k[i].numel(), kv.v[i].numel()))
        check(lib().flyai_stage_set_layer(self._h, i, C.byref(d)))
        self.layers[i] = lw

    def set_workspace(self):
        """Bind a freshly allocated device workspace (and the pinned staging).  Drops every captured
        step graph."""
        dev_bytes = int(lib().flyai_stage_workspace_bytes(self._h))
        ws = torch.empty(dev_bytes + 256, dtype=torch.uint8, device=self.device)
        ptr = ws.data_ptr() + (-ws.data_ptr()) % 256
        check(lib().flyai_stage_set_workspace(self._h, C.c_void_p(ptr), dev_bytes,
                                              C.c_void_p(self.staging.data_ptr()), self.staging.numel()))
        self.workspace, self._ws_ptr = ws, ptr

    def set_graphs(self, enable):
        """Replay each step as a HIP graph, one per (tokens, sequences, attention-plan bucket), captured
        on first use (the CUDA-graph capture of FastVerify.decode, phase0/fastverify.py:221-231)."""
        if bool(enable) != self.use_graphs:
            check(lib().flyai_stage_set_graphs(self._h, int(bool(enable))))
            self.use_graphs = bool(enable)

    @property
    def graphs_captured(self):
        return int(lib().flyai_stage_graphs_captured(self._h))

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._h = None
            try:
                self._sync(self.device)
            except Exception:
                pass
            self._destroy(h)

    def forward(self, hidden, q_lens, starts, slots):
        """hidden bf16 [T, H] (packed token order, updated in place and returned); q_lens/starts/slots
        per sequence (host ints).  Raises ContextOverflow before any write."""
        S = len(q_lens)
        if not (len(starts) == S == len(slots)):
            raise ValueError("q_lens, starts and slots must have one entry per sequence")
        T = int(sum(int(q) for q in q_lens))
        if hidden.dtype != torch.bfloat16 or not hidden.is_contiguous() or tuple(hidden.shape) != (T, self.shape.hidden):
            raise ValueError(f"hidden must be contiguous bf16 [{T}, {self.shape.hidden}]")
        for s in slots:
            if not 0 <= int(s) < self.kv.n_slots:
                raise ValueError(f"slot {s} out of range")
        if len(set(int(s) for s in slots)) != S:
            raise ValueError("two sequences of one step share a KV slot (their K/V writes would race)")
        ql = np.ascontiguousarray(q_lens, dtype=np.int32)
        st = np.ascontiguousarray(starts, dtype=np.int32)
        base = np.ascontiguousarray([self.kv.base(int(s)) for s in slots], dtype=np.int64)
        cap = np.ascontiguousarray([self.kv.slot_cap(int(s)) for s in slots], dtype=np.int32)
        lim = np.asarray([self.kv.maxlens[int(s)] for s in slots], dtype=np.int64)
        need = st.astype(np.int64) + ql
        if np.any(need > lim):
            b = int(np.argmax(need > lim))
            raise ContextOverflow(_lib.FLYAI_ERANGE, f"sequence {b} needs {int(need[b])} positions > max_ctx {int(lim[b])}")
        check(lib().flyai_stage_forward(
            self._h, ql.ctypes.data_as(C.c_void_p), st.ctypes.data_as(C.c_void_p),
            base.ctypes.data_as(C.c_void_p), cap.ctypes.data_as(C.c_void_p), S,
            C.c_void_p(hidden.data_ptr()), C.c_void_p(torch.cuda.current_stream(self.device).cuda_stream)))
        return hidden

    def forward_tree(self, hidden, start, par, dep, slot=0):
        """Tree verify of one sequence (``FastVerify.tree_decode``, phase0/fastverify.py:281-299):
        hidden bf16 [M, H] holds the M tree nodes (updated in place and returned); node i is rotated
        at position start + dep[i], its K/V goes to slot start + i and it attends the committed
        prefix and its ancestors.  The caller validates the tree (``validate_tree``)."""
        M = len(par)
        if hidden.dtype != torch.bfloat16 or not hidden.is_contiguous() or tuple(hidden.shape) != (M, self.shape.hidden):
            raise ValueError(f"hidden must be contiguous bf16 [{M}, {self.shape.hidden}]")
        if not 0 <= int(slot) < self.kv.n_slots:
            raise ValueError(f"slot {slot} out of range")
        pa = np.ascontiguousarray(par, dtype=np.int32)
        de = np.ascontiguousarray(dep, dtype=np.int32)
        check(lib().flyai_stage_forward_tree(
            self._h, int(start), M, pa.ctypes.data_as(C.c_void_p), de.ctypes.data_as(C.c_void_p),
            self.kv.base(int(slot)), self.kv.slot_cap(int(slot)), C.c_void_p(hidden.data_ptr()),
            C.c_void_p(torch.cuda.current_stream(self.device).cuda_stream)))
        return hidden

    def debug_buffer(self, which, dtype, shape):
        """A view of an internal buffer of the last step (tests only); see flyai_stage.h."""
        ptr = lib().flyai_stage_debug_buffer(self._h, which)
        off = ptr - self.workspace.data_ptr()
        n = int(np.prod(shape)) * torch.tensor([], dtype=dtype).element_size()
        return self.workspace[off:off + n].view(dtype).view(*shape)


TREE_MAX_NODES = 2048  # FLYAI_TREE_MAX_NODES: the stage reserves the masks of a tree this large


def validate_tree(M, par, dep):
    """Reject a malformed tree before any parent walk (``validate_tree``, phase0/fastverify.py:29-49):
    par/dep are M long; every parent is an int in [-1, M) and not the node itself; depths are
    non-negative ints with dep[i] == 0 for a root and dep[par[i]] + 1 otherwise (which rules out
    cycles).  Raises ValueError."""
    if not isinstance(M, int) or isinstance(M, bool) or M < 1:
        raise ValueError(f"tree size {M!r} invalid")
    if len(par) != M or len(dep) != M:
        raise ValueError(f"tree par/dep lengths {len(par)}/{len(dep)} != {M} nodes")
    for i in range(M):
        p, d = par[i], dep[i]
        if not isinstance(p, int) or isinstance(p, bool) or not (-1 <= p < M) or p == i:
            raise ValueError(f"tree node {i}: parent {p!r} out of range [-1, {M})")
        if not isinstance(d, int) or isinstance(d, bool) or d < 0:
            raise ValueError(f"tree node {i}: depth {d!r} invalid")
    for i in range(M):
        want = 0 if par[i] == -1 else dep[par[i]] + 1
        if dep[i] != want:
            raise ValueError(f"tree node {i}: depth {dep[i]} != {want} (parent {par[i]}; cycle or bad depth)")


class FastVerifyStage:
    """Drop-in for ``FastVerify(parts, maxlen, dev)`` (phase0/fastverify.py:80-309), B = 1.

    ``parts`` is the reference's dict: either what ``flyai_amd.stage_parts.load_stage`` returns or the
    reference's own (transformers modules, converted by ``stage_parts.parts_from_reference``).  Keys
    read: ``layers``, ``rotary``, ``sliding`` (carried by each layer), ``_model.config`` or ``shape``.
    ``decode`` returns a buffer the runtime owns and reuses on the next call (as the graph output is
    in the reference)."""

    DECODE_BUCKETS = (2048, 4096, 8192, 16384, 32768, 65536, 131072)

    def __init__(self, parts, maxlen=2048, dev="cuda", max_tokens=4096):
        parts = stage_parts.as_stage_parts(parts, dev)
        self.parts, self.maxlen, self.dev = parts, maxlen, dev
        self.shape = stage_parts.stage_shape(parts)
        self.layers = parts["layers"]
        self.n_layers = len(self.layers)
        self.hidden = self.shape.hidden
        self.cache = KVWorkspace(self.n_layers, 1, maxlen, self.shape.n_kv_heads, self.shape.head_dim, dev)
        self.stage = RaggedStage(self.shape, self.layers, parts["rotary"], self.cache, max_tokens, 1, device=dev)
        self.out = None

    def reset(self):
        self.cache.zero()

    def _run(self, h, start):
        n = h.shape[1]
        if start + n > self.maxlen:
            raise ContextOverflow(_lib.FLYAI_ERANGE, f"needs {start + n} positions > max_ctx {self.maxlen} (raise --max-ctx)")
        flat = h.reshape(n, self.hidden).to(torch.bfloat16).contiguous().clone()
        self.stage.forward(flat, [n], [start], [0])
        return flat.view(1, n, self.hidden)

    def prefill(self, h, start):
        self.stage.set_graphs(False)  # prefill runs eager in the reference (fastverify.py:138-155)
        return self._run(h, start)

    def decode(self, h, start):
        self.stage.set_graphs(True)  # one graph per (tokens, KV bucket), as fastverify.py:221-231
        self.out = self._run(h, start)
        return self.out

    def tree_decode(self, h, start, par, dep):
        """Verify a fixed-topology tree of M nodes in one pass (fastverify.py:281-299): node i at
        position start + dep[i], K/V at scratch slot start + i, attending the committed prefix and its
        ancestors.  Malformed trees raise ValueError and overflows ContextOverflow, both before any
        write.  Trees are limited to min(max_tokens, 2048) nodes (ValueError beyond)."""
        M = h.shape[1]
        validate_tree(M, list(par), list(dep))
        if start + M > self.maxlen:
            raise ContextOverflow(_lib.FLYAI_ERANGE, f"tree decode needs {start + M} positions > max_ctx "
                                  f"{self.maxlen} (raise --max-ctx)")
        limit = min(TREE_MAX_NODES, self.stage.max_tokens)
        if M > limit:
            raise ValueError(f"tree of {M} nodes exceeds the {limit}-node limit")
        self.stage.set_graphs(False)
        flat = h.reshape(M, self.hidden).to(torch.bfloat16).contiguous().clone()
        self.stage.forward_tree(flat, start, list(par), list(dep), 0)
        self.tout = flat.view(1, M, self.hidden)
        return self.tout

    def tree_gather(self, start, keep):
        """Compact the accepted path's KV (scratch slots start+keep[i]) to start+i, every layer
        (fastverify.py:301-309)."""
        src = torch.tensor([start + k for k in keep], device=self.dev)
        dst = torch.arange(start, start + len(keep), device=self.dev)
        for l in range(self.n_layers):
            self.cache.move_positions(l, 0, src, dst)


class BatchedFastVerifyStage:
    """Drop-in for ``BatchedFastVerify(parts, B, maxlen, dev)`` (phase0/batchverify.py:64-190).

    Every stream is one ragged sequence of kp1 tokens at its own start; per-stream KV slabs and the
    per-row order-fixed MoE make each stream's output independent of its batch mates."""

    DECODE_BUCKETS = FastVerifyStage.DECODE_BUCKETS

    def __init__(self, parts, B, maxlen=2048, dev="cuda", lossless=False, max_tokens=None):
        parts = stage_parts.as_stage_parts(parts, dev)
        self.parts, self.B, self.maxlen, self.dev = parts, B, maxlen, dev
        self.shape = stage_parts.stage_shape(parts)
        self.layers = parts["layers"]
        self.n_layers = len(self.layers)
        self.hidden = self.shape.hidden
        self.cache = KVWorkspace(self.n_layers, B, maxlen, self.shape.n_kv_heads, self.shape.head_dim, dev)
        self.stage = RaggedStage(self.shape, self.layers, parts["rotary"], self.cache,
                                 max_tokens or 64 * B, B, device=dev)
        self.out = None

    def reset(self):
        self.cache.zero()

    def load_prefix(self, b, src_cache):
        """Copy a solo runtime's committed KV (its KVWorkspace, slot 0) into stream b."""
        self.cache.copy_slot(b, src_cache, 0)

    def decode(self, h, starts, use_graph=True):
        B, kp1, H = h.shape
        if B != self.B:
            raise ValueError(f"expected {self.B} streams, got {B}")
        st = [int(v) for v in (starts.tolist() if torch.is_tensor(starts) else starts)]
        need = max(st) + kp1
        if need > self.maxlen:
            raise ContextOverflow(_lib.FLYAI_ERANGE, f"batched decode needs {need} positions > max_ctx {self.maxlen}")
        flat = h.reshape(B * kp1, H).to(torch.bfloat16).contiguous().clone()
        self.stage.set_graphs(use_graph)
        self.stage.forward(flat, [kp1] * B, st, list(range(B)))
        self.out = flat.view(B, kp1, H)
        return self.out


class Fp8MoeStage:
    """A stage of DeepSeek-V3-shaped FP8 MoE layers over a flat ragged token batch: per layer
    h += MoE(RMSNorm(h)) with grouped sigmoid routing, FP8 routed experts and the shared expert
    (vendor/deepseek_v4_ref/inference/model.py:634-650 MoE, :592-611 Expert).  Every op is a
    libflyai_stage launch on the current stream."""

    def __init__(self, shape, layers):
        self.shape, self.layers = shape, layers

    def moe(self, lw, x, residual):
        sh = self.shape
        T = x.shape[0]
        E, k, H, I = sh.n_experts, sh.top_k, sh.hidden, sh.intermediate
        xn = ops.rmsnorm(x, lw.ln, sh.rms_eps)
        ids, wts, _ = ops.router_grouped_sigmoid(xn, lw.router_w, lw.e_bias, sh.n_group, sh.topk_group, k,
                                                 sh.route_scale)
        _, off, perm, inv = ops.moe_permute(ids, E)
        xq, xs = ops.fp8_act_quant(xn)
        # routed rows 0..P-1 then the shared expert's T rows, in one launch per projection
        h = ops.moe_gate_up_fp8(xq, xs, perm, off, k, wts, lw.w13_packed, E, I, n_shared=T)
        hq, hs = ops.fp8_act_quant(h)
        y = ops.moe_down_fp8(hq, hs, off, lw.w2_packed, E, H, n_shared=T)
        P = T * k
        return ops.moe_combine_sum(y[:P], inv, k, shared=y[P:], residual=residual, out=residual)

    def forward(self, hidden):
        """hidden bf16 [T, H], updated in place through every layer."""
        for lw in self.layers:
            self.moe(lw, hidden, hidden)
        return hidden
