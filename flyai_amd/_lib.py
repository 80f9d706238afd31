"""ctypes binding of libflyai_stage.so (the gfx950 HIP library built by flyai_amd.build).

There is no fallback: if the library is missing or fails to load, every entry point raises."""
import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libflyai_stage.so")

FLYAI_OK, FLYAI_EINVAL, FLYAI_ERANGE, FLYAI_EHIP = 0, -1, -2, -3


class FlyaiError(RuntimeError):
    """A C-ABI call returned an error code."""

    def __init__(self, code, msg):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class ContextOverflow(FlyaiError):
    """A sequence needs more KV positions than its workspace holds (phase0/fastverify.py:23-26)."""


class AttnItem(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("seq", "kv_head", "tok", "ntok", "pos0", "key_lo", "key_hi", "group")]


class AttnGroup(C.Structure):
    _fields_ = [("first_item", C.c_int32), ("n_splits", C.c_int32), ("tok", C.c_int32),
                ("ntok", C.c_int32), ("kv_head", C.c_int32), ("pad", C.c_int32 * 3)]


class StageConfig(C.Structure):
    _fields_ = [(n, C.c_int32) for n in (
        "n_layers", "hidden", "n_q_heads", "n_kv_heads", "head_dim", "n_experts", "top_k",
        "intermediate", "window", "max_tokens", "max_seqs", "max_attn_items", "rope_positions",
        "attn_split_keys")] + [("rms_eps", C.c_float), ("attn_prefill_min", C.c_int32),
                               ("moe_dense_fp8", C.c_int32)]


class LayerDesc(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in (
        "ln1", "ln2", "wqkv", "bqkv", "wo", "bo", "sinks", "router_w", "router_b", "w13_packed",
        "b13", "w2_packed", "b2", "k_pool", "v_pool")] + [("sliding", C.c_int32), ("pad", C.c_int32),
                                                          ("kv_pool_elems", C.c_int64)]


P, I32, I64, F32, SZ = C.c_void_p, C.c_int32, C.c_int64, C.c_float, C.c_size_t

# name -> (restype, argtypes)
_PROTOS = {
    "flyai_last_error": (C.c_char_p, []),
    "flyai_abi_version": (C.c_int, []),
    "flyai_pack_ragged": (C.c_int, [P, P, P, P, I32, I32, I32, P, P, P, P, P, P, P]),
    "flyai_router_topk_softmax": (C.c_int, [P, P, P, I32, I32, I32, I32, P, P, P, P]),
    "flyai_moe_permute": (C.c_int, [P, I32, I32, I32, P, P, P, P, P]),
    "flyai_moe_route_permute": (C.c_int, [P, P, P, I32, I32, I32, I32, P, P, P, P, P, P, P, P]),
    "flyai_moe_combine": (C.c_int, [P, P, P, I32, I32, I32, P, P, P]),
    "flyai_router_grouped_sigmoid": (C.c_int, [P, P, P, I32, I32, I32, I32, I32, I32, F32, P, P, P, P]),
    "flyai_fp8_act_quant": (C.c_int, [P, I32, I32, P, P, P]),
    "flyai_fp8_packed_bytes": (SZ, [I32, I32, I32]),
    "flyai_fp8_repack": (C.c_int, [P, P, P, P, I32, I32, I32, P, P]),
    "flyai_moe_gate_up_fp8": (C.c_int, [P, P, P, P, I32, P, P, I32, I32, I32, I32, P, P]),
    "flyai_moe_down_fp8": (C.c_int, [P, P, P, P, I32, I32, I32, I32, P, P]),
    "flyai_moe_combine_sum": (C.c_int, [P, P, I32, I32, I32, P, P, P, P]),
    "flyai_mxfp4_packed_bytes": (SZ, [I32, I32, I32]),
    "flyai_mxfp4_repack": (C.c_int, [P, P, I32, I32, I32, P, P]),
    "flyai_moe_gate_up_mxfp4": (C.c_int, [P, P, P, I32, I32, P, P, I32, I32, I32, P, P]),
    "flyai_moe_down_mxfp4": (C.c_int, [P, P, I32, P, P, I32, I32, I32, P, P]),
    "flyai_mx_act_scale_bytes": (SZ, [I32, I32]),
    "flyai_mx_act_quant": (C.c_int, [P, I32, I32, P, P, P]),
    "flyai_moe_gate_up_mxfp4_fp8act": (C.c_int, [P, P, P, P, P, I32, I32, P, P, I32, I32, I32, P, P]),
    "flyai_moe_down_mxfp4_fp8act": (C.c_int, [P, P, P, P, I32, P, P, I32, I32, I32, P, P]),
    "flyai_rmsnorm": (C.c_int, [P, P, I32, I32, F32, P, P]),
    "flyai_linear_workspace_bytes": (SZ, [I32, I32, I32]),
    "flyai_linear_bf16": (C.c_int, [P, P, P, I32, I32, I32, P, P, P, P]),
    "flyai_linear_noalloc_max_bytes": (SZ, []),
    "flyai_linear_bf16_noalloc": (C.c_int, [P, P, P, I32, I32, I32, P, P, P]),
    "flyai_rope_kv_append": (C.c_int, [P, P, P, P, P, I32, I32, I32, I32, I32, P, P, P, P, P, P]),
    "flyai_attn_plan": (C.c_int, [P, P, I32, I32, I32, I32, P, I32, P, I32, P, P, P]),
    "flyai_attn_partials_bytes": (SZ, [I32]),
    "flyai_attn_plan_prefill": (C.c_int, [P, P, I32, I32, I32, I32, I32, P, I32, P, I32, P, I32, P, P, P, P]),
    "flyai_attn_prefill": (C.c_int, [P, P, P, P, P, P, I32, I32, I32, I32, P, I32, P, P]),
    "flyai_attn_ragged": (C.c_int, [P, P, P, P, P, P, I32, I32, I32, I32, P, I32, I32, P, I32, P, P, P]),
    "flyai_bf16_tile_packed_bytes": (SZ, [I32, I32]),
    "flyai_bf16_tile_repack": (C.c_int, [P, I32, I32, P, P]),
    "flyai_embed_gather": (C.c_int, [P, P, I32, I32, I32, P, P]),
    "flyai_lm_head_workspace_bytes": (SZ, [I32, I32]),
    "flyai_lm_head_argmax": (C.c_int, [P, P, I32, I32, P, I32, P, P, P, P]),
    "flyai_hbm_read_probe": (C.c_int, [P, SZ, I32, I32, P, P]),
    "flyai_sample_rows": (C.c_int, [P, I32, I32, F32, I32, F32, P, P, P, P, P, P]),
    "flyai_sample_probs": (C.c_int, [P, I32, C.c_double, P, P]),
    "flyai_stage_create": (C.c_int, [P, P]),
    "flyai_stage_destroy": (None, [P]),
    "flyai_stage_set_layer": (C.c_int, [P, I32, P]),
    "flyai_stage_set_rope": (C.c_int, [P, P, P]),
    "flyai_stage_workspace_bytes": (SZ, [P]),
    "flyai_stage_host_staging_bytes": (SZ, [P]),
    "flyai_stage_set_workspace": (C.c_int, [P, P, SZ, P, SZ]),
    "flyai_stage_forward": (C.c_int, [P, P, P, P, P, I32, P, P]),
    "flyai_stage_forward_tree": (C.c_int, [P, I32, I32, P, P, I64, I32, P, P]),
    "flyai_stage_debug_buffer": (P, [P, I32]),
    "flyai_stage_set_graphs": (C.c_int, [P, I32]),
    "flyai_stage_graphs_captured": (I32, [P]),
}

_lib = None


def lib():
    """Load the library once; raise if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FlyaiError(FLYAI_EINVAL, f"{LIB_PATH} is not built; run `python -m flyai_amd.build`")
        handle = C.CDLL(LIB_PATH)
        for name, (res, args) in _PROTOS.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def exported_names():
    return list(_PROTOS)


def check(rc):
    if rc != FLYAI_OK:
        msg = lib().flyai_last_error().decode(errors="replace")
        if rc == FLYAI_ERANGE:
            raise ContextOverflow(rc, msg)
        raise FlyaiError(rc, msg)
    return rc
