"""The tiled KV slab layout (flyai_amd.kvlayout, the host twin of kv_k_off / kv_v_off in
csrc/common.h): a bijection per head region, and exactly the order in which the attention kernel's
lanes consume each 64-key block (no GPU needed)."""
import torch

from flyai_amd import kvlayout


def tile_key(kt, m):
    return 32 * (kt // 2) + 8 * (m // 4) + 4 * (kt % 2) + m % 4


def test_offsets_are_a_bijection_per_head_region():
    cap = 192
    pos = torch.arange(cap)
    for fn in (kvlayout.k_offsets, kvlayout.v_offsets):
        off = fn(pos).reshape(-1)
        assert torch.equal(torch.sort(off).values, torch.arange(cap * 64))


def test_k_blocks_follow_the_kernels_fragment_order():
    """Block b, 16-byte piece (kt, step, lane = 16 gd + n): key 64 b + tile_key(kt, n), dims
    32 step + 8 gd .. +7 -- what load_k_tile reads at blk + kt*1024 + step*512 + lane*8."""
    for b in (0, 3):
        for kt in range(4):
            for step in range(2):
                for lane in (0, 5, 16, 37, 63):
                    gd, n = lane // 16, lane % 16
                    key = 64 * b + tile_key(kt, n)
                    dims = torch.arange(32 * step + 8 * gd, 32 * step + 8 * gd + 8)
                    want = b * 4096 + kt * 1024 + step * 512 + lane * 8 + torch.arange(8)
                    assert torch.equal(kvlayout.k_offsets(torch.tensor([key]))[0, dims], want)


def test_v_blocks_follow_the_kernels_fragment_order():
    """Block b, piece (h, dt, lane = 16 gk + n): dim 16 dt + n, keys 64 b + 32 h + 8 gk .. +7 -- what
    load_v_tile reads at blk + h*2048 + dt*512 + lane*8."""
    for b in (0, 2):
        for h in range(2):
            for dt in range(4):
                for lane in (0, 9, 31, 48, 63):
                    gk, n = lane // 16, lane % 16
                    keys = 64 * b + 32 * h + 8 * gk + torch.arange(8)
                    want = b * 4096 + h * 2048 + dt * 512 + lane * 8 + torch.arange(8)
                    assert torch.equal(kvlayout.v_offsets(keys)[:, 16 * dt + n], want)


def test_pack_gather_scatter_roundtrip():
    g = torch.Generator().manual_seed(0)
    Hkv, cap = 3, 128
    k = torch.randn(Hkv, cap, 64, generator=g)
    flat = kvlayout.pack(k, "k")
    assert torch.equal(kvlayout.gather(flat, Hkv, cap, "k"), k)
    pos = torch.tensor([5, 70, 127])
    new = torch.randn(Hkv, 3, 64, generator=g)
    kvlayout.scatter(flat, Hkv, cap, "k", new, pos)
    k[:, pos] = new
    assert torch.equal(kvlayout.gather(flat, Hkv, cap, "k"), k)
    v = torch.randn(2, Hkv, cap, 64, generator=g)
    vflat = kvlayout.pack(v, "v")
    assert torch.equal(kvlayout.gather(vflat[1], Hkv, cap, "v"), v[1])


def test_workspace_with_per_slot_capacities():
    """A per-sequence workspace: slot i holds caps[i] positions (rounded up to 64), slabs back to back;
    dense writes and reads go through each slot's own capacity."""
    import torch
    from flyai_amd.runtime import KVWorkspace
    kv = KVWorkspace(2, 3, 0, 2, 64, device="cpu", caps=[100, 64, 200])
    assert kv.caps == [128, 64, 256] and kv.maxlens == [100, 64, 200] and kv.cap == 256
    assert [kv.base(s) for s in range(3)] == [0, 2 * 128 * 64, 2 * (128 + 64) * 64]
    assert kv.k[0].numel() == 2 * (128 + 64 + 256) * 64
    g = torch.Generator().manual_seed(3)
    for slot, n in ((0, 100), (2, 200)):
        k = torch.randn(2, n, 64, generator=g).to(torch.bfloat16)
        v = torch.randn(2, n, 64, generator=g).to(torch.bfloat16)
        kv.set_dense(1, slot, k, v, positions=list(range(n)))
        assert torch.equal(kv.k_dense(1, slot, positions=list(range(n))), k)
        assert torch.equal(kv.v_dense(1, slot, positions=list(range(n))), v)
    assert kv.k[1][kv.base(1):kv.base(2)].abs().sum() == 0      # slot 1 untouched
