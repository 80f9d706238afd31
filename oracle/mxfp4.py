"""MXFP4 block format: packed E2M1 codes with one E8M0 scale per 32 values (row a5).

Follows ``transformers/integrations/mxfp4.py``:
  * ``FP4_VALUES`` code table, ``mxfp4.py:29-46``;
  * ``_convert_moe_packed_tensors``, ``mxfp4.py:257-313``: value = LUT[nibble] * 2**(scale-127),
    the LOW nibble of byte i is element 2i and the high nibble element 2i+1 (``:298-304``);
  * expert parameter layout ``Mxfp4GptOssExperts``, ``mxfp4.py:349-365``:
    gate_up blocks [E, 2I, H/32, 16] u8, scales [E, 2I, H/32] u8, bias [E, 2I] fp32;
    down    blocks [E, H, I/32, 16] u8,  scales [E, H, I/32] u8,  bias [E, H] fp32.

Unlike the HF helper (which transposes to [E, in, out] for ``x @ W``), ``dequant`` keeps the
stored orientation: row n of the result is output feature n, so ``y = x @ W.T``.

E8M0 byte 255 is NaN (OCP MX v1.0 section 5.4); every value scaled by it is NaN.  Byte 0 is
2**-127.  Parity: closed form, exhaustively checked over all 256 code bytes x all 256 scale bytes
against the transformers fixture (tests/golden) and against the table below.
"""
import numpy as np
import torch

# mxfp4.py:29-46, in code order 0..15 (codes 8..15 are the negatives, sign = bit 3).
FP4_VALUES = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
              -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0)
LUT = np.array(FP4_VALUES, dtype=np.float32)
# byte -> (value of low nibble, value of high nibble): element 2i then 2i+1
PAIR_LUT = np.stack([LUT[np.arange(256) & 0x0F], LUT[np.arange(256) >> 4]], axis=-1)


def e8m0_to_f32(s):
    """E8M0 byte(s) -> float32: 2**(s-127); 255 -> NaN."""
    s = np.asarray(s, dtype=np.int32)
    out = np.ldexp(np.ones(s.shape, dtype=np.float32), s - 127).astype(np.float32)
    out = np.where(s == 255, np.float32(np.nan), out)
    return out.astype(np.float32)


_PAIR_LUT_T = torch.from_numpy(PAIR_LUT)


def dequant(blocks, scales):
    """blocks u8 [..., G, 16], scales u8 [..., G] -> float32 [..., G*32] (exact).  The table lookup
    and the power-of-two scaling run as torch CPU ops, which use every intra-op thread."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    scales = np.asarray(scales, dtype=np.uint8)
    assert blocks.shape[:-1] == scales.shape and blocks.shape[-1] == 16
    vals = _PAIR_LUT_T[torch.from_numpy(blocks).long()].reshape(*blocks.shape[:-1], 32)  # low nibble first
    vals *= torch.from_numpy(e8m0_to_f32(scales))[..., None]
    return vals.reshape(*blocks.shape[:-2], blocks.shape[-2] * 32).numpy()


def dequant_rows(blocks, scales, rows):
    """Dequantize only the listed output rows of one expert: blocks [N, G, 16] -> [len(rows), K]."""
    return dequant(blocks[rows], scales[rows])
