"""GPT-OSS yarn rotary tables (the stage's ``parts["rotary"]``).

Follows ``_compute_yarn_parameters`` (transformers/modeling_rope_utils.py:345-483) with the GPT-OSS
defaults (configuration_gpt_oss.py:29, :80-88) and ``GptOssRotaryEmbedding.forward``
(modeling_gpt_oss.py:189-200): cos/sin of fp32 ``inv_freq * position`` times ``attention_scaling``,
rounded to bf16.  The table is computed once on the host with torch's fp32 CPU ops (the same
operation sequence transformers uses, so the bf16 values are identical) and kept on the GPU,
where the RoPE kernel indexes it by position -- a constant, like a weight."""
import math

import torch


class YarnRotary:
    @classmethod
    def from_inv_freq(cls, inv_freq, attention_scaling, n_positions, device="cuda"):
        """The table of a rotary module that already holds its fp32 inv_freq and attention_scaling
        (transformers' GptOssRotaryEmbedding): the same product, cos/sin, scaling and bf16 rounding."""
        self = cls.__new__(cls)
        self.inv_freq = inv_freq.detach().float().cpu()
        self.attention_scaling = float(attention_scaling)
        self.head_dim = 2 * self.inv_freq.numel()
        self._tables(n_positions, device)
        return self

    def _tables(self, n_positions, device):
        self.n_positions = n_positions
        pos = torch.arange(n_positions, dtype=torch.float32)
        freqs = (self.inv_freq[None, :, None] @ pos[None, None, :]).transpose(1, 2)[0]
        self.cos = (freqs.cos() * self.attention_scaling).to(torch.bfloat16).contiguous().to(device)
        self.sin = (freqs.sin() * self.attention_scaling).to(torch.bfloat16).contiguous().to(device)

    def __init__(self, n_positions, head_dim=64, base=150000.0, factor=32.0, beta_fast=32.0,
                 beta_slow=1.0, original_max=4096, truncate=False, device="cuda"):
        dim = head_dim
        att = 1.0 if factor <= 1 else 0.1 * math.log(factor) + 1.0

        def corr(num_rot):
            return (dim * math.log(original_max / (num_rot * 2 * math.pi))) / (2 * math.log(base))

        low, high = corr(beta_fast), corr(beta_slow)
        if truncate:
            low, high = math.floor(low), math.ceil(high)
        low, high = max(low, 0), min(high, dim - 1)
        if low == high:
            high += 0.001
        ramp = torch.clamp((torch.arange(dim // 2, dtype=torch.float32) - low) / (high - low), 0, 1)
        pos_freqs = base ** (torch.arange(0, dim, 2).to(dtype=torch.float) / dim)
        extra = 1 - ramp
        self.inv_freq = (1.0 / (factor * pos_freqs)) * (1 - extra) + (1.0 / pos_freqs) * extra
        self.attention_scaling = att
        self.head_dim = head_dim
        self._tables(n_positions, device)
