"""The KV slab layout the attention kernel reads (the host twin of kv_k_off / kv_v_off in
csrc/common.h), with gathers between it and dense [Hkv, cap, 64] tensors.

Per kv head, a region of cap x 64 bf16 (cap % 64 == 0) in 64-key blocks of 4096 elements, each in
MFMA-fragment order so that one 16-byte load per lane of a wave reads one contiguous KiB:

* K: [kt 4][step 2][lane 64][8]: lane 16*gd + n holds key tile_key(kt, n) of the block and dims
  32*step + 8*gd .. +7, with tile_key(kt, m) = 32*(kt//2) + 8*(m//4) + 4*(kt%2) + m%4;
* V: [h 2][dt 4][lane 64][8]: lane 16*gk + n holds dim 16*dt + n and keys 32*h + 8*gk .. +7.

A slab is Hkv consecutive head regions.  The layout replaces StaticKV's [1, Hkv, maxlen, D] and
BatchedStaticKV's [B, Hkv, maxlen, D] (phase0/fastverify.py:52-77, phase0/batchverify.py:29-48)."""
import torch

HEAD_DIM = 64


def k_offsets(positions):
    """Element offsets [P, 64] of key rows (positions: int64 tensor) within a head region."""
    p = positions.long()[:, None]
    d = torch.arange(HEAD_DIM, device=p.device)[None, :]
    kk = p % 64
    kt = 2 * (kk // 32) + (kk % 8) // 4
    n = 4 * ((kk % 32) // 8) + kk % 4
    return (p // 64) * 4096 + kt * 1024 + (d // 32) * 512 + (16 * ((d % 32) // 8) + n) * 8 + d % 8


def v_offsets(positions):
    """Element offsets [P, 64] of value rows within a head region."""
    p = positions.long()[:, None]
    d = torch.arange(HEAD_DIM, device=p.device)[None, :]
    kk = p % 64
    return (p // 64) * 4096 + (kk // 32) * 2048 + (d // 16) * 512 + (16 * ((kk % 32) // 8) + d % 16) * 8 + kk % 8


def _index(offsets_fn, n_heads, cap, positions, device):
    pos = torch.as_tensor(positions, device=device).long() if positions is not None else torch.arange(cap, device=device)
    heads = torch.arange(n_heads, device=device)[:, None, None] * (cap * HEAD_DIM)
    return heads + offsets_fn(pos)[None]                                   # [Hkv, P, 64]


def gather(flat_slab, n_heads, cap, kind, positions=None):
    """Dense [Hkv, P, 64] copy of a slab's K ("k") or V ("v") rows (all positions by default)."""
    fn = k_offsets if kind == "k" else v_offsets
    return flat_slab[_index(fn, n_heads, cap, positions, flat_slab.device)]


def scatter(flat_slab, n_heads, cap, kind, dense, positions=None):
    """Write dense [Hkv, P, 64] rows into a slab (all positions by default)."""
    fn = k_offsets if kind == "k" else v_offsets
    flat_slab[_index(fn, n_heads, cap, positions, flat_slab.device)] = dense.to(flat_slab.dtype)


def pack(dense, kind):
    """Dense [..., Hkv, cap, 64] -> flat tiled slabs [..., Hkv * cap * 64]."""
    *lead, n_heads, cap, _ = dense.shape
    flat = torch.empty(*lead, n_heads * cap * HEAD_DIM, dtype=dense.dtype, device=dense.device)
    fn = k_offsets if kind == "k" else v_offsets
    idx = _index(fn, n_heads, cap, None, dense.device)
    flat[..., idx.reshape(-1)] = dense.reshape(*lead, -1)
    return flat
