"""GPT-OSS MXFP4 checkpoint loading into the stage's layout, with a fail-closed layout guard.

The reference loads GPT-OSS through transformers' MXFP4 quantizer and then verifies the loaded
storage with ``inspect_mxfp4_quantized`` (``phase0/mxfp4_guard.py:279-359``, per projection
``_packed_projection`` ``:223-276``).  Here the same rules are applied to the checkpoint's own
safetensors storage, before anything reaches the GPU, and the verified tensors are then loaded
layer by layer into ``LayerWeights``: the MXFP4 experts re-packed by ``flyai_mxfp4_repack``,
q/k/v stacked, norms, sinks and expert biases in fp32.

Checkpoint names (the HF GPT-OSS layout, ``transformers/integrations/mxfp4.py:349-365``), per layer
``model.layers.{i}.``:
  ``mlp.experts.{gate_up,down}_proj_{blocks,scales,bias}``  blocks u8 [E, rows, cols/32, 16],
      scales u8 / E8M0 [E, rows, cols/32], bias [E, rows]; gate_up rows 2I x cols H, down H x I
  ``mlp.router.{weight,bias}``, ``self_attn.{q,k,v,o}_proj.{weight,bias}``, ``self_attn.sinks``,
  ``input_layernorm.weight``, ``post_attention_layernorm.weight``;
and ``model.embed_tokens.weight``, ``model.norm.weight``, ``lm_head.weight`` for the head and tail.

A checkpoint is one ``.safetensors`` file or a directory with ``model.safetensors`` or a
``model.safetensors.index.json`` weight map.  Tensors are opened lazily (``safe_open``); only the
assigned layers are read.
"""
import json
import os

import torch
from safetensors import safe_open

from .weights import GptOssShape, LayerWeights

PROJECTIONS = ("gate_up_proj", "down_proj")
SCALE_DTYPES = ("U8", "F8_E8M0")
EXPERT_TENSORS = tuple(p + s for p in PROJECTIONS for s in ("_blocks", "_scales", "_bias"))


class MXFP4LayoutError(ValueError):
    """The checkpoint's storage is not the packed MXFP4 layout the stage reads (fail closed)."""


class CheckpointReader:
    """Lazy access to the tensors of a safetensors checkpoint (one file, or shards + index)."""

    def __init__(self, path):
        if os.path.isdir(path):
            index = os.path.join(path, "model.safetensors.index.json")
            if os.path.exists(index):
                with open(index) as f:
                    weight_map = json.load(f)["weight_map"]
                self.files = {name: os.path.join(path, fn) for name, fn in weight_map.items()}
            else:
                single = os.path.join(path, "model.safetensors")
                if not os.path.exists(single):
                    raise FileNotFoundError(f"no model.safetensors or index in {path}")
                self.files = self._names_of(single)
        else:
            self.files = self._names_of(path)
        cfg = os.path.join(path if os.path.isdir(path) else os.path.dirname(path), "config.json")
        self.config = None
        if os.path.exists(cfg):
            with open(cfg) as f:
                self.config = json.load(f)
        self._handles = {}

    @staticmethod
    def _names_of(fn):
        with safe_open(fn, framework="pt") as f:
            return {name: fn for name in f.keys()}

    def _handle(self, fn):
        if fn not in self._handles:
            self._handles[fn] = safe_open(fn, framework="pt")
        return self._handles[fn]

    def keys(self):
        return self.files.keys()

    def __contains__(self, name):
        return name in self.files

    def meta(self, name):
        """(dtype string, shape tuple) without reading the data."""
        sl = self._handle(self.files[name]).get_slice(name)
        return sl.get_dtype(), tuple(sl.get_shape())

    def get(self, name, device="cpu"):
        return self._handle(self.files[name]).get_tensor(name).to(device)


def check_quantization_config(config):
    """The checkpoint must declare native MXFP4 storage and must not ask for dequantization (the
    reference's ``config_uses_mxfp4`` and its refusal of a dequantizing quantizer,
    ``phase0/mxfp4_guard.py``)."""
    q = (config or {}).get("quantization_config") or {}
    if q.get("quant_method") != "mxfp4":
        raise MXFP4LayoutError("checkpoint config does not declare real MXFP4 quantization")
    if q.get("dequantize"):
        raise MXFP4LayoutError("checkpoint config asks for a dequantized fallback")


def shape_from_config(config):
    """(GptOssShape, number of decoder layers, per-layer sliding flags) from a GPT-OSS config.json."""
    c = config
    shape = GptOssShape(hidden=c["hidden_size"], intermediate=c["intermediate_size"],
                        n_experts=c["num_local_experts"],
                        top_k=c.get("num_experts_per_tok", c.get("experts_per_token", 4)),
                        n_q_heads=c["num_attention_heads"], n_kv_heads=c["num_key_value_heads"],
                        head_dim=c.get("head_dim", 64), window=c.get("sliding_window", 128),
                        rms_eps=c.get("rms_norm_eps", 1e-5))
    n = c["num_hidden_layers"]
    types = c.get("layer_types") or ["sliding_attention" if i % 2 == 0 else "full_attention" for i in range(n)]
    if len(types) != n:
        raise MXFP4LayoutError("layer_types does not match num_hidden_layers")
    return shape, n, [t == "sliding_attention" for t in types]


def _layer_indices(reader):
    idx = set()
    for name in reader.keys():
        if name.startswith("model.layers."):
            part = name.split(".")[2]
            if not part.isdigit():
                raise MXFP4LayoutError(f"unexpected decoder-layer tensor name {name}")
            idx.add(int(part))
    return idx


def _expect(reader, name, shape=None, dtypes=None, what=None):
    if name not in reader:
        raise MXFP4LayoutError(f"missing {what or name}")
    dtype, got = reader.meta(name)
    if dtypes is not None and dtype not in dtypes:
        raise MXFP4LayoutError(f"{name} has dtype {dtype}, expected one of {dtypes}")
    if shape is not None and got != tuple(shape):
        raise MXFP4LayoutError(f"{name} has shape {got}, expected {tuple(shape)}")
    return dtype, got


def inspect_mxfp4_checkpoint(reader, shape, n_layers, layer_range=None):
    """Verify the packed MXFP4 expert layout of the assigned layers, and every other tensor the stage
    reads, from storage metadata alone (``inspect_mxfp4_quantized`` rules): the declared layer count,
    the assigned range, expert dimensions in blocks of 32, u8 blocks [E, rows, cols/32, 16] and E8M0
    byte scales [E, rows, cols/32] per projection, biases [E, rows], and no expanded floating-point
    expert matrix beside the packed ones (the expert module holds exactly the six packed tensors).
    When the reader carries a config.json its quantization declaration is checked too.  Raises
    MXFP4LayoutError; returns a report like the reference's."""
    if reader.config is not None:
        check_quantization_config(reader.config)
    E, H, I = shape.n_experts, shape.hidden, shape.intermediate
    if H % 32 or I % 32:
        raise MXFP4LayoutError("MXFP4 expert dimensions require blocks of 32")
    present = _layer_indices(reader)
    if present != set(range(len(present))) or len(present) != n_layers:
        raise MXFP4LayoutError(f"checkpoint has decoder layers {sorted(present)[:4]}..., expected {n_layers}")
    lo, hi = layer_range if layer_range is not None else (0, n_layers)
    if type(lo) is not int or type(hi) is not int or not 0 <= lo < hi <= n_layers:
        raise MXFP4LayoutError("invalid assigned MXFP4 layer range")
    nq, nkv = shape.n_q_heads * shape.head_dim, shape.n_kv_heads * shape.head_dim
    observed, packed_bytes = [], 0
    for i in range(lo, hi):
        p = f"model.layers.{i}."
        for proj in PROJECTIONS:
            rows, cols = (2 * I, H) if proj == "gate_up_proj" else (H, I)
            base = p + "mlp.experts." + proj
            _expect(reader, base + "_blocks", (E, rows, cols // 32, 16), ("U8",), f"packed expert {proj}")
            _expect(reader, base + "_scales", (E, rows, cols // 32), SCALE_DTYPES, f"{proj} block scales")
            _expect(reader, base + "_bias", (E, rows), None, f"{proj} bias")
            packed_bytes += E * rows * cols // 2 + E * rows * cols // 32
        for name in reader.keys():  # nothing expanded or unconverted may hide beside the packed experts
            if name.startswith(p + "mlp.experts.") and name[len(p) + 12:] not in EXPERT_TENSORS:
                raise MXFP4LayoutError(f"unconverted expert tensor {name} ({reader.meta(name)[0]}) is present")
        _expect(reader, p + "mlp.router.weight", (E, H))
        _expect(reader, p + "mlp.router.bias", (E,))
        for proj, (n_out, n_in) in (("q_proj", (nq, H)), ("k_proj", (nkv, H)), ("v_proj", (nkv, H)),
                                    ("o_proj", (H, nq))):
            _expect(reader, p + f"self_attn.{proj}.weight", (n_out, n_in))
            _expect(reader, p + f"self_attn.{proj}.bias", (n_out,))
        _expect(reader, p + "self_attn.sinks", (shape.n_q_heads,))
        _expect(reader, p + "input_layernorm.weight", (H,))
        _expect(reader, p + "post_attention_layernorm.weight", (H,))
        observed.append({"layer": i, "module": "mlp.experts"})
    return {"packed_layout_verified": True, "native_execution_verified": False, "layer_range": [lo, hi], "experts": observed,
            "packed_weight_scale_bytes": packed_bytes,
            "scope": "checkpoint storage layout only; kernel output is validated separately"}


def load_stage_layers(reader, shape, layer_range, device="cuda", sliding=None, keep_hf=False):
    """LayerWeights of layers [lo, hi) on `device`, MXFP4 experts re-packed for the stage.  Layer i
    uses the sliding window iff sliding[i] (default: the config's layer_types, else GPT-OSS's
    alternation starting with a sliding layer).  Run inspect_mxfp4_checkpoint first."""
    lo, hi = layer_range
    if sliding is None:
        sliding = (shape_from_config(reader.config)[2] if reader.config is not None
                   else [i % 2 == 0 for i in range(hi)])
    out = []
    for i in range(lo, hi):
        p = f"model.layers.{i}."

        def get(name, dtype):
            return reader.get(p + name, device).to(dtype).contiguous()

        bf, f32 = torch.bfloat16, torch.float32
        scales = {proj: reader.get(p + f"mlp.experts.{proj}_scales", device) for proj in PROJECTIONS}
        scales = {k: (v.view(torch.uint8) if v.dtype != torch.uint8 else v).contiguous() for k, v in scales.items()}
        lw = LayerWeights(
            ln1=get("input_layernorm.weight", f32), ln2=get("post_attention_layernorm.weight", f32),
            wqkv=torch.cat([get(f"self_attn.{n}.weight", bf) for n in ("q_proj", "k_proj", "v_proj")]).contiguous(),
            bqkv=torch.cat([get(f"self_attn.{n}.bias", bf) for n in ("q_proj", "k_proj", "v_proj")]).contiguous(),
            wo=get("self_attn.o_proj.weight", bf), bo=get("self_attn.o_proj.bias", bf),
            sinks=get("self_attn.sinks", f32),
            router_w=get("mlp.router.weight", bf), router_b=get("mlp.router.bias", bf),
            w13_blocks=get("mlp.experts.gate_up_proj_blocks", torch.uint8), w13_scales=scales["gate_up_proj"],
            b13=get("mlp.experts.gate_up_proj_bias", f32),
            w2_blocks=get("mlp.experts.down_proj_blocks", torch.uint8), w2_scales=scales["down_proj"],
            b2=get("mlp.experts.down_proj_bias", f32),
            sliding=bool(sliding[i]))
        out.append(lw.repack(keep_hf=keep_hf))
    return out


def load_head_tail(reader, device="cuda", tie_word_embeddings=False):
    """(embed bf16 [V, H], final norm fp32 [H], lm_head bf16 [V, H]) for GptOssModel."""
    embed = reader.get("model.embed_tokens.weight", device).to(torch.bfloat16).contiguous()
    norm = reader.get("model.norm.weight", device).float().contiguous()
    lm = embed if tie_word_embeddings else reader.get("lm_head.weight", device).to(torch.bfloat16).contiguous()
    return embed, norm, lm
