"""Rounding helpers shared by the oracle modules (test infrastructure only)."""
import numpy as np
import torch


def bf16(x):
    """Round an fp32 tensor to bfloat16 (round-to-nearest-even) and return it as fp32.

    torch's float->bfloat16 cast is RNE, the same rounding the reference's bf16 tensors get
    from every Linear/add in ``transformers/models/gpt_oss/modeling_gpt_oss.py``."""
    return x.float().to(torch.bfloat16).float()


def bf16_bits_to_f32(u16):
    """uint16 bfloat16 bit patterns (numpy) -> float32 numpy array (exact)."""
    return (np.asarray(u16, dtype=np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x):
    """float32 numpy array -> uint16 bfloat16 bits, round-to-nearest-even (NaN kept quiet)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    out = rounded.astype(np.uint16)
    out[nan] = 0x7FC0
    return out
