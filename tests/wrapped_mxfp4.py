"""Stand-ins for the kernel library's wrapped MXFP4 expert tensors, for the parts adapter's tests.

Native MXFP4 loading in transformers (what the reference's ``load_stage`` requires,
``phase0/pipeline.py:147-160``) replaces each expert projection's parameter with a wrapper object:
``.storage.data`` holds the physical uint8 bytes in a hardware-specific swizzle, ``.storage.layout``
can undo it (``unswizzle_data``), ``.shape`` is the transposed logical shape [E, K, N] and ``.dtype``
names FP4; the E8M0 scales ride in ``<proj>_precision_config.weight_scale``, wrapped the same way
(``transformers/integrations/mxfp4.py:603-649`` builds them, ``:203-222`` reverses them).

The kernel library is not installed here, so ``TiledLayout`` is a swizzle of this file's own: it pads
the two last axes to whole tiles and stores the tiles N-major with each tile transposed, which moves
every byte that can move.  ``unswizzle_data`` is its exact inverse.  ``keep_padding`` makes the
inverse return the padded array, as a layout may."""
import torch


class FP4:
    """The wrapper's dtype: the adapter only needs ``"fp4"`` in its name."""

    def __repr__(self):
        return "FP4"


class TiledLayout:
    def __init__(self, shape, tk=8, tn=32, keep_padding=False):
        self.E, self.K, self.N = shape
        self.tk, self.tn, self.keep_padding = tk, tn, keep_padding
        self.Kp = -(-self.K // tk) * tk
        self.Np = -(-self.N // tn) * tn

    def swizzle_data(self, data):
        assert tuple(data.shape) == (self.E, self.K, self.N)
        pad = torch.zeros(self.E, self.Kp, self.Np, dtype=data.dtype, device=data.device)
        pad[:, :self.K, :self.N] = data
        t = pad.view(self.E, self.Kp // self.tk, self.tk, self.Np // self.tn, self.tn)
        t = t.permute(0, 3, 1, 4, 2).contiguous()          # [E, N tiles, K tiles, tn, tk]
        return t.view(self.E, -1, self.tn * self.tk)

    def unswizzle_data(self, data):
        t = data.reshape(self.E, self.Np // self.tn, self.Kp // self.tk, self.tn, self.tk)
        t = t.permute(0, 2, 4, 1, 3).contiguous().view(self.E, self.Kp, self.Np)
        return t if self.keep_padding else t[:, :self.K, :self.N]


class Storage:
    def __init__(self, data, layout):
        self.data, self.layout = data, layout


class WrappedTensor:
    def __init__(self, data, logical_shape, layout, dtype):
        self.storage = Storage(layout.swizzle_data(data), layout)
        self.shape = torch.Size(logical_shape)
        self.dtype = dtype


class PrecisionConfig:
    def __init__(self, weight_scale):
        self.weight_scale = weight_scale


def wrap_projection(experts, proj, blocks, scales, keep_padding=False, tk=8, tn=32):
    """Replace ``<proj>_blocks`` / ``<proj>_scales`` on `experts` by the wrapped form, the way native
    loading does: codes transposed to [E, cols/2, rows] bytes (two fp4 per byte along K) with the
    logical shape [E, cols, rows], scales transposed to [E, cols/32, rows]."""
    E, rows, kg, _ = blocks.shape
    cols = kg * 32
    codes = blocks.reshape(E, rows, cols // 2).transpose(1, 2).contiguous()
    sc = scales.view(torch.uint8).transpose(1, 2).contiguous()
    w = WrappedTensor(codes, (E, cols, rows), TiledLayout(codes.shape, tk, tn, keep_padding), FP4())
    s = WrappedTensor(sc, (E, cols // 32, rows), TiledLayout(sc.shape, 2, tn, keep_padding), torch.uint8)
    for name in (proj + "_blocks", proj + "_scales", proj):
        if name in experts._parameters:
            del experts._parameters[name]
        elif hasattr(experts, name):
            delattr(experts, name)
    object.__setattr__(experts, proj, w)
    object.__setattr__(experts, proj + "_precision_config", PrecisionConfig(s))
    return w, s
