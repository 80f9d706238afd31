"""The reference's stage ``parts`` dict, served by libflyai_stage.

The reference's serve loops build their stage from ``parts = load_stage(...)``
(``phase0/pipeline.py:126-182``) and then read, per role:

* every stage: ``FastVerify(parts, maxlen, dev)`` (``phase0/specpipe.py:544``, ``:666``), which takes
  ``parts["layers"]``, ``["rotary"]``, ``["sliding"]``, ``["window"]`` and ``["_model"].config``
  (``phase0/fastverify.py:85-91``); ``parts["lo"]`` / ``["hi"]`` for receipts;
* the head: ``parts["embed"](ids)`` (``specpipe.py:596``);
* the tail: ``parts["norm"](h)`` and ``parts["lm_head"](h)`` (``specpipe.py:611-612``, ``:796``).

Two ways to get such a dict here:

* ``load_stage(model_id, stage, nstages, device, dtype, attn, lo, hi)`` -- the reference's signature,
  reading a local GPT-OSS MXFP4 safetensors checkpoint directory (``flyai_amd.checkpoint``, behind the
  MXFP4 layout guard) straight into the stage's layout;
* ``parts_from_reference(parts)`` -- converts a dict whose ``layers`` are transformers
  ``GptOssDecoderLayer`` modules (what the reference's ``load_stage`` returns) by reading the modules'
  own parameters: ``input_layernorm``, ``post_attention_layernorm``, ``self_attn.{q,k,v,o}_proj``,
  ``self_attn.sinks``, ``mlp.router`` and the packed MXFP4 experts with their ``<proj>_bias``.  The
  experts may hold the wrapped tensors native MXFP4 loading leaves (``<proj>`` with
  ``<proj>_precision_config``, the form the reference's ``load_stage`` produces), ``<proj>_blocks`` /
  ``<proj>_scales``, or raw ``<proj>`` bytes with ``<proj>_scales``.

Either way the dict keeps the reference's keys, and ``embed`` / ``norm`` / ``lm_head`` are callables
over the HIP kernels (``flyai_embed_gather``, ``flyai_rmsnorm``, ``flyai_lm_head_argmax``).  The
stage runtimes (``FastVerifyStage``, ``BatchedFastVerifyStage``) accept both dicts."""
import types

import torch

from . import ops
from .checkpoint import (CheckpointReader, MXFP4LayoutError, check_quantization_config, inspect_mxfp4_checkpoint,
                         load_head_tail, load_stage_layers, shape_from_config)
from .rope import YarnRotary
from .weights import GptOssShape, LayerWeights

LM_HEAD_ROWS = 64   # rows per lm_head launch (the kernel's limit)


# ---- head and tail callables ---------------------------------------------------------------------

class Embedding:
    """``parts["embed"]``: token ids (any integer tensor, [..., n]) -> bf16 hidden rows [..., n, H]."""

    def __init__(self, weight):
        self.weight = ops._need(weight.to(torch.bfloat16).contiguous(), torch.bfloat16, name="embedding")
        self.vocab, self.hidden = self.weight.shape

    def __call__(self, ids):
        ids = torch.as_tensor(ids, device=self.weight.device)
        flat = ids.reshape(-1).to(torch.int32).contiguous()
        out = ops.embed_gather(self.weight, flat)
        return out.view(*ids.shape, self.hidden)


class FinalNorm:
    """``parts["norm"]``: the final RMSNorm, bf16 [..., H] -> bf16 [..., H] (fp32 weight)."""

    def __init__(self, weight, eps=1e-5):
        self.weight, self.eps = weight.float().contiguous(), float(eps)

    def __call__(self, h):
        H = h.shape[-1]
        flat = h.reshape(-1, H).to(torch.bfloat16).contiguous()
        return ops.rmsnorm(flat, self.weight, self.eps).view(h.shape)


class LmHead:
    """``parts["lm_head"]``: normed bf16 rows [..., n, H] -> bf16 logits [..., n, V].  The nn.Linear weight
    [V, H] is re-packed once into the lm_head kernel's tile layout; ``argmax`` gives the greedy ids
    without materialising the logits."""

    def __init__(self, weight):
        w = weight.to(torch.bfloat16).contiguous()
        self.vocab, self.hidden = w.shape
        self.packed = ops.bf16_tile_repack(w)

    def _rows(self, h):
        return h.reshape(-1, self.hidden).to(torch.bfloat16).contiguous()

    def __call__(self, h):
        x = self._rows(h)
        out = torch.empty(x.shape[0], self.vocab, dtype=torch.bfloat16, device=x.device)
        for r0 in range(0, x.shape[0], LM_HEAD_ROWS):
            rows = x[r0:r0 + LM_HEAD_ROWS].contiguous()
            _, logits = ops.lm_head_argmax(rows, self.packed, self.vocab, want_logits=True)
            out[r0:r0 + rows.shape[0]] = logits
        return out.view(*h.shape[:-1], self.vocab)

    def argmax(self, h):
        x = self._rows(h)
        ids = [ops.lm_head_argmax(x[r0:r0 + LM_HEAD_ROWS].contiguous(), self.packed, self.vocab)
               for r0 in range(0, x.shape[0], LM_HEAD_ROWS)]
        return torch.cat(ids).view(*h.shape[:-1])


class _Config(types.SimpleNamespace):
    """Attribute view of a config.json dict (what the runtimes read as ``parts["_model"].config``)."""


class _ModelHandle:
    def __init__(self, config):
        self.config = config


def _config_dict(config):
    if isinstance(config, dict):
        return dict(config)
    if hasattr(config, "to_dict"):
        return config.to_dict()
    return dict(vars(config))


def stage_shape(parts):
    """GptOssShape of a parts dict: ``parts["shape"]`` when present, else from ``_model.config``."""
    if parts.get("shape") is not None:
        return parts["shape"]
    model = parts.get("_model")
    if model is not None and getattr(model, "config", None) is not None:
        return shape_from_config(_config_dict(model.config))[0]
    return GptOssShape()


# ---- layers from transformers modules ----------------------------------------------------------

def _param(module, path):
    obj = module
    for name in path.split("."):
        obj = getattr(obj, name, None)
        if obj is None:
            raise MXFP4LayoutError(f"decoder layer has no {path}")
    return obj.detach() if torch.is_tensor(obj) else obj


def _is_wrapped(value):
    """A kernel-library tensor wrapper (what transformers attaches on native MXFP4 loading): an object,
    not a torch tensor, whose ``storage`` holds the physical bytes in ``data`` and their ``layout``."""
    storage = getattr(value, "storage", None)
    return not torch.is_tensor(value) and torch.is_tensor(getattr(storage, "data", None))


def _unswizzled(value, what, logical, packed, padded, dtypes):
    """The bytes of a wrapped tensor in its logical, unswizzled [E, K-side, N] order.

    The checks restate the reference guard's for the wrapped form (``phase0/mxfp4_guard.py:232-243``,
    ``:264-267``): the published logical shape, the physical byte count between the packed and the
    512-padded size, and the storage dtype.  The layout object undoes its own swizzle
    (``storage.layout.unswizzle_data``, the call transformers' reverse op makes,
    ``transformers/integrations/mxfp4.py:203-222``); nothing of the kernel library is imported here.
    A layout that keeps its padding after unswizzling has it cut from the ends of the last two axes."""
    if tuple(getattr(value, "shape", ())) != tuple(logical):
        raise MXFP4LayoutError(f"{what} has logical shape {tuple(getattr(value, 'shape', ()))}, "
                               f"expected {tuple(logical)}")
    data = value.storage.data
    if data.dtype not in dtypes:
        raise MXFP4LayoutError(f"{what} storage holds {data.dtype}, not packed bytes")
    nbytes = data.numel() * data.element_size()
    if not packed <= nbytes <= padded:
        raise MXFP4LayoutError(f"{what} storage has {nbytes} bytes, outside [{packed}, {padded}]")
    unswizzle = getattr(getattr(value.storage, "layout", None), "unswizzle_data", None)
    if unswizzle is None:
        raise MXFP4LayoutError(f"{what} storage layout has no unswizzle_data")
    out = unswizzle(data)
    E, k, n = logical[0], packed // (logical[0] * logical[2]), logical[2]
    if not torch.is_tensor(out) or out.dim() != 3 or out.shape[0] != E or out.shape[1] < k or out.shape[2] < n:
        raise MXFP4LayoutError(f"{what} unswizzles to {tuple(getattr(out, 'shape', ()))}, expected {(E, k, n)}")
    if out.dtype != torch.uint8:
        out = out.view(torch.uint8)
    return out[:, :k, :n]


def _wrapped_storage(experts, proj, rows, cols, n_experts):
    """(blocks, scales) of a wrapped projection, in the raw checkpoint layout.

    The wrapper publishes the transposed logical shape [E, cols, rows] (K before N) and stores the
    fp4 codes two per byte along K; its scales ride in ``<proj>_precision_config.weight_scale`` with
    logical shape [E, cols/32, rows].  Transposing the unswizzled bytes back gives the checkpoint's
    [E, rows, cols/2] codes and [E, rows, cols/32] scales (transformers' reverse op, ``mxfp4.py:203-222``)."""
    raw = getattr(experts, proj)
    if not ("fp4" in str(getattr(raw, "dtype", "")).lower()):
        raise MXFP4LayoutError(f"experts.{proj} wrapper is not FP4 ({getattr(raw, 'dtype', None)})")
    logical = (n_experts, cols, rows)
    packed = n_experts * rows * cols // 2
    padded = n_experts * -(-cols // 512) * 512 * -(-rows // 512) * 512 // 2
    codes = _unswizzled(raw, f"experts.{proj}", logical, packed, padded, (torch.uint8,))
    scale = getattr(getattr(experts, proj + "_precision_config", None), "weight_scale", None)
    if scale is None:
        raise MXFP4LayoutError(f"experts.{proj}_precision_config has no weight_scale")
    sdt = tuple(t for t in (torch.uint8, getattr(torch, "float8_e8m0fnu", None)) if t is not None)
    slogical = (n_experts, cols // 32, rows)
    if _is_wrapped(scale):
        sbytes = _unswizzled(scale, f"experts.{proj} weight_scale", slogical, packed // 16, padded // 16, sdt)
    else:
        if not torch.is_tensor(scale) or tuple(scale.shape) != slogical or scale.dtype not in sdt:
            raise MXFP4LayoutError(f"experts.{proj} weight_scale is not E8M0 bytes of shape {slogical}")
        sbytes = scale.view(torch.uint8)
    blocks = codes.detach().transpose(1, 2).contiguous().reshape(n_experts, rows, cols // 32, 16)
    scales = sbytes.detach().transpose(1, 2).contiguous()
    return blocks, scales


def _expert_storage(experts, proj, rows, cols, n_experts):
    """(blocks u8 [E, rows, cols/32, 16], scales u8 [E, rows, cols/32]) of one packed projection:
    ``<proj>_blocks`` + ``<proj>_scales`` (before the load swizzle), raw ``<proj>`` bytes +
    ``<proj>_scales``, or the wrapped ``<proj>`` + ``<proj>_precision_config`` that native MXFP4 loading
    leaves (``phase0/pipeline.py:147-160``)."""
    if getattr(experts, proj + "_blocks", None) is None and _is_wrapped(getattr(experts, proj, None)):
        return _wrapped_storage(experts, proj, rows, cols, n_experts)
    blocks = getattr(experts, proj + "_blocks", None)
    if blocks is None:
        blocks = getattr(experts, proj, None)
    scales = getattr(experts, proj + "_scales", None)
    if not torch.is_tensor(blocks) or not torch.is_tensor(scales):
        raise MXFP4LayoutError(
            f"experts.{proj} is neither packed MXFP4 with {proj}_scales nor a wrapped MXFP4 tensor (a "
            "dequantized expert cannot be re-packed); load the stage with flyai_amd.stage_parts.load_stage instead")
    blocks, scales = blocks.detach(), scales.detach()
    if blocks.dtype != torch.uint8:
        raise MXFP4LayoutError(f"experts.{proj} holds {blocks.dtype}, not packed E2M1 bytes")
    if tuple(blocks.shape) == (n_experts, rows, cols // 2):
        blocks = blocks.reshape(n_experts, rows, cols // 32, 16)
    if tuple(blocks.shape) != (n_experts, rows, cols // 32, 16):
        raise MXFP4LayoutError(f"experts.{proj} has shape {tuple(blocks.shape)}, expected "
                               f"{(n_experts, rows, cols // 32, 16)}")
    if scales.dtype != torch.uint8:
        scales = scales.view(torch.uint8)
    if tuple(scales.shape) != (n_experts, rows, cols // 32):
        raise MXFP4LayoutError(f"experts.{proj}_scales has shape {tuple(scales.shape)}, expected "
                               f"{(n_experts, rows, cols // 32)}")
    return blocks, scales


def module_tensors(layer, shape: GptOssShape, sliding, device="cpu"):
    """The stage's tensors of one transformers GptOssDecoderLayer, before the MXFP4 re-pack: the
    LayerWeights fields with q/k/v stacked on the output axis, norms, sinks and expert biases in fp32,
    the packed experts as HF-layout blocks [E, rows, cols/32, 16] and scale bytes [E, rows, cols/32]."""
    E, H, I = shape.n_experts, shape.hidden, shape.intermediate
    nq, nkv = shape.n_q_heads * shape.head_dim, shape.n_kv_heads * shape.head_dim
    bf, f32 = torch.bfloat16, torch.float32

    def get(path, dtype, want):
        t = _param(layer, path)
        if tuple(t.shape) != tuple(want):
            raise MXFP4LayoutError(f"{path} has shape {tuple(t.shape)}, expected {tuple(want)}")
        return t.to(device=device, dtype=dtype).contiguous()

    ex = _param(layer, "mlp.experts")
    w13, s13 = _expert_storage(ex, "gate_up_proj", 2 * I, H, E)
    w2, s2 = _expert_storage(ex, "down_proj", H, I, E)
    qkv = (("q_proj", nq), ("k_proj", nkv), ("v_proj", nkv))
    return dict(
        ln1=get("input_layernorm.weight", f32, (H,)), ln2=get("post_attention_layernorm.weight", f32, (H,)),
        wqkv=torch.cat([get(f"self_attn.{p}.weight", bf, (n, H)) for p, n in qkv]).contiguous(),
        bqkv=torch.cat([get(f"self_attn.{p}.bias", bf, (n,)) for p, n in qkv]).contiguous(),
        wo=get("self_attn.o_proj.weight", bf, (H, nq)), bo=get("self_attn.o_proj.bias", bf, (H,)),
        sinks=get("self_attn.sinks", f32, (shape.n_q_heads,)),
        router_w=get("mlp.router.weight", bf, (E, H)), router_b=get("mlp.router.bias", bf, (E,)),
        w13_blocks=w13.to(device).contiguous(), w13_scales=s13.to(device).contiguous(),
        b13=get("mlp.experts.gate_up_proj_bias", f32, (E, 2 * I)),
        w2_blocks=w2.to(device).contiguous(), w2_scales=s2.to(device).contiguous(),
        b2=get("mlp.experts.down_proj_bias", f32, (E, H)),
        sliding=bool(sliding))


def layer_from_module(layer, shape: GptOssShape, sliding, device="cuda", keep_hf=False):
    """LayerWeights of one transformers GptOssDecoderLayer, its MXFP4 experts re-packed on `device`."""
    return LayerWeights(**module_tensors(layer, shape, sliding, device)).repack(keep_hf=keep_hf)


def _rotary_from(module, n_positions, head_dim, config, device):
    """The stage's rope table.  A transformers rotary module carries its inv_freq and
    attention_scaling, and the table is computed from them exactly as its forward does; otherwise
    the yarn parameters come from the config's rope_scaling."""
    inv = getattr(module, "inv_freq", None)
    att = getattr(module, "attention_scaling", None)
    if torch.is_tensor(inv) and att is not None:
        return YarnRotary.from_inv_freq(inv.detach().float().cpu(), float(att), n_positions, device=device)
    rs = config.get("rope_scaling") or config.get("rope_parameters") or {}
    base = rs.get("rope_theta") or config.get("rope_theta") or 150000.0
    return YarnRotary(n_positions, head_dim=head_dim, base=base,
                      factor=rs.get("factor", 32.0), beta_fast=rs.get("beta_fast", 32.0),
                      beta_slow=rs.get("beta_slow", 1.0),
                      original_max=rs.get("original_max_position_embeddings", 4096),
                      truncate=rs.get("truncate", False), device=device)


def _positions(config, n_positions):
    return int(n_positions or config.get("max_position_embeddings") or 131072)


def parts_from_reference(parts, device="cuda", n_positions=None, keep_hf=False):
    """The reference's parts dict (transformers modules) -> the same keys over the HIP library."""
    model = parts.get("_model")
    if model is None or getattr(model, "config", None) is None:
        raise ValueError("parts needs '_model' with a config (what the reference's load_stage returns)")
    cfg = _config_dict(model.config)
    shape, n_total, _ = shape_from_config(cfg)
    mods = list(parts["layers"])
    sliding = parts.get("sliding")
    if sliding is None:
        sliding = [False] * len(mods)
    layers = [layer_from_module(m, shape, sliding[i], device, keep_hf) for i, m in enumerate(mods)]
    out = {"layers": layers, "shape": shape, "_model": model, "sliding": list(sliding),
           "window": parts.get("window", shape.window), "n_layers": parts.get("n_layers", n_total),
           "lo": parts.get("lo", 0), "hi": parts.get("hi", len(layers)),
           "rotary": _rotary_from(parts.get("rotary"), _positions(cfg, n_positions), shape.head_dim, cfg, device)}
    if parts.get("embed") is not None:
        out["embed"] = Embedding(_param(parts["embed"], "weight").to(device))
    if parts.get("norm") is not None:
        out["norm"] = FinalNorm(_param(parts["norm"], "weight").to(device), shape.rms_eps)
    if parts.get("lm_head") is not None:
        out["lm_head"] = LmHead(_param(parts["lm_head"], "weight").to(device))
    return out


def as_stage_parts(parts, device="cuda"):
    """``parts`` ready for the stage runtimes: a dict of LayerWeights passes through (with its shape
    filled in); a dict of transformers layers is converted by parts_from_reference."""
    layers = parts["layers"]
    if len(layers) and not isinstance(layers[0], LayerWeights):
        return parts_from_reference(parts, device)
    if parts.get("shape") is None:
        parts = dict(parts, shape=stage_shape(parts))
    return parts


# ---- straight from a checkpoint -------------------------------------------------------------------

def load_stage(model_id, stage, nstages, device="cuda", dtype="auto", attn="eager", lo=None, hi=None,
               n_positions=None):
    """``load_stage`` (phase0/pipeline.py:126-182) over a local GPT-OSS MXFP4 checkpoint directory:
    layers [lo, hi) of stage `stage` of `nstages` (even split by default), the embedding on the head
    (stage 0) and the final norm and lm_head on the tail.  The checkpoint's config must declare MXFP4
    and its storage passes the layout guard before any tensor reaches the GPU.  dtype must be "auto"
    or bfloat16 (the stage computes in the checkpoint's own precision); attn is accepted for the
    signature's sake (the stage has one attention kernel)."""
    if dtype not in ("auto", torch.bfloat16, "bfloat16"):
        raise ValueError(f"dtype {dtype!r}: the stage runs the checkpoint's MXFP4/bf16 weights as stored")
    reader = CheckpointReader(model_id)
    if reader.config is None:
        raise FileNotFoundError(f"{model_id} has no config.json")
    cfg = reader.config
    check_quantization_config(cfg)
    shape, n_layers, sliding_all = shape_from_config(cfg)
    if not (isinstance(stage, int) and isinstance(nstages, int) and 0 <= stage < nstages):
        raise ValueError(f"stage {stage!r} of {nstages!r}")
    if lo is None or hi is None:
        lo, hi = stage * n_layers // nstages, (stage + 1) * n_layers // nstages
    inspect_mxfp4_checkpoint(reader, shape, n_layers, layer_range=(lo, hi))
    layers = load_stage_layers(reader, shape, (lo, hi), device=device, sliding=sliding_all)
    window = cfg.get("sliding_window", 0) or 0
    parts = {"layers": layers, "shape": shape, "n_layers": n_layers, "lo": lo, "hi": hi,
             "_model": _ModelHandle(_Config(**cfg)), "window": window,
             "sliding": [sliding_all[j] for j in range(lo, hi)] if window else None,
             "rotary": _rotary_from(None, _positions(cfg, n_positions), shape.head_dim, cfg, device)}
    is_head, is_tail = stage == 0, stage == nstages - 1
    if is_head or is_tail:
        embed, norm_w, lm_w = load_head_tail(reader, device, bool(cfg.get("tie_word_embeddings", False)))
        if is_head:
            parts["embed"] = Embedding(embed)
        if is_tail:
            parts["norm"] = FinalNorm(norm_w, shape.rms_eps)
            parts["lm_head"] = LmHead(lm_w)
    return parts
