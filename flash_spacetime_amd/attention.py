"""Model-side caller: `Attention_rel`-shaped multi-head attention on the fused op.

graphnet reaches the reference operator through `Block_rel.forward_flash`
(reference README.md:105-116): the module projects q, k and v with
`proj_q`, `proj_k`, `proj_v` (and optional `q_bias`, `v_bias`), splits the
heads, calls `flash_spacetime_attention`, merges the heads and applies its
output projection `proj` (the parameter names `attention_rel_oracle_inputs`
reads, reference.py:198-223). The reference's op then copies the split views
to contiguous `[B, H, L, D]` (forward.py:274) and the merge copies the output
back to `[B, L, H*D]`.

Here self-attention projects q, k and v with one GEMM (`proj_q`, `proj_k`,
`proj_v` stacked into one `[3*H*D, dim]` weight) whose `[B, L, 3*H*D]`
output, viewed as `[B, L, 3, H, D]`, is what `flash_spacetime_attention_qkv`
reads in place; its gradient comes back as one tensor of that layout, which
the same linear's backward consumes. The output is `[B, L, H, D]`, so
merging the heads is free. Nothing is transposed, split, stacked or copied
around the fused op in either direction. Cross-attention (a separate `kv`)
uses three linears whose split heads are token-major views, also read in
place.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import Tensor, nn
from torch.nn import functional as F

from .reference import merge_heads, split_heads


class SpacetimeAttention(nn.Module):
    """Multi-head self-attention with the spacetime pair bias.

    Parameters follow graphnet's `Attention_rel`: `proj_q`, `proj_k`,
    `proj_v` (no bias), `q_bias` / `v_bias` when `qkv_bias`, `proj` (output),
    `num_heads`. `rel_proj` is the pair-embedding projection `R = E W^T + b`
    of the operator (`weight [D, C]`, `bias [D]`, nn.Linear layout).
    `forward(x, feats, seqlens | key_padding_mask)` takes `x [B, L, dim]`,
    detector features `feats [B, L, F >= 4]` and the event lengths, and
    returns `[B, L, dim]`; with `cu_seqlens` it takes packed events, `x
    [T, dim]` and `feats [T, F]`, and returns `[T, dim]`.
    """

    def __init__(self, dim: int, num_heads: int = 8, channels: int = 16, qkv_bias: bool = False,
                 head_dim: Optional[int] = None, use_attn_bias: bool = True,
                 use_activation_bias: bool = True, device=None, dtype=None) -> None:
        super().__init__()
        fk = {"device": device, "dtype": dtype}
        self.num_heads = num_heads
        self.head_dim = head_dim if head_dim is not None else dim // num_heads
        inner = self.head_dim * num_heads
        self.proj_q = nn.Linear(dim, inner, bias=False, **fk)
        self.proj_k = nn.Linear(dim, inner, bias=False, **fk)
        self.proj_v = nn.Linear(dim, inner, bias=False, **fk)
        if qkv_bias:
            self.q_bias = nn.Parameter(torch.zeros(inner, **fk))
            self.v_bias = nn.Parameter(torch.zeros(inner, **fk))
        else:
            self.q_bias = None
            self.v_bias = None
        self.rel_proj = nn.Linear(channels, self.head_dim, **fk)
        self.proj = nn.Linear(inner, dim, **fk)
        self.use_attn_bias = use_attn_bias
        self.use_activation_bias = use_activation_bias

    def qkv_weight(self) -> Tuple[Tensor, Optional[Tensor]]:
        """The stacked `[3*H*D, dim]` projection weight and its bias (k has none)."""
        w = torch.cat((self.proj_q.weight, self.proj_k.weight, self.proj_v.weight))
        if self.q_bias is None:
            return w, None
        return w, torch.cat((self.q_bias, torch.zeros_like(self.q_bias), self.v_bias))

    def project_qkv(self, x: Tensor, kv: Optional[Tensor] = None) -> Tuple[Tensor, Tensor, Tensor]:
        """q, k, v `[B, H, L, D]` with the values of `attention_rel_oracle_inputs`.

        Self-attention: heads-first views of the one fused projection
        (`[B, L, 3, H, D]`); with a separate `kv`: token-major views of three
        linears.
        """
        b, length, _ = x.shape
        if kv is None:
            w, bias = self.qkv_weight()
            qkv = F.linear(x, w, bias).view(b, length, 3, self.num_heads, self.head_dim)
            return tuple(qkv[:, :, i].transpose(1, 2) for i in range(3))
        if kv.shape != x.shape:
            raise ValueError(f"kv must have the shape of x {tuple(x.shape)}, got {tuple(kv.shape)}")
        q = F.linear(x, self.proj_q.weight, self.q_bias)
        k = F.linear(kv, self.proj_k.weight)
        v = F.linear(kv, self.proj_v.weight, self.v_bias)
        return tuple(split_heads(t, self.num_heads) for t in (q, k, v))

    def forward(self, x: Tensor, feats: Tensor, seqlens: Optional[Tensor] = None,
                key_padding_mask: Optional[Tensor] = None, kv: Optional[Tensor] = None,
                cu_seqlens: Optional[Tensor] = None) -> Tensor:
        from .forward import flash_spacetime_attention, flash_spacetime_attention_qkv

        flags = (self.use_attn_bias, self.use_activation_bias)
        if cu_seqlens is not None:
            if kv is not None or seqlens is not None or key_padding_mask is not None:
                raise ValueError("packed input takes cu_seqlens only (self-attention, no lengths or mask)")
            if x.dim() != 2:
                raise ValueError(f"packed x must be [T, dim], got {tuple(x.shape)}")
            w, bias = self.qkv_weight()
            qkv = F.linear(x, w, bias).view(x.shape[0], 3, self.num_heads, self.head_dim)
            out = flash_spacetime_attention_qkv(qkv, feats, self.rel_proj.weight, self.rel_proj.bias, None, None,
                                                *flags, cu_seqlens=cu_seqlens)
            return self.proj(out.reshape(x.shape[0], -1))
        b, length, _ = x.shape
        if kv is None:
            w, bias = self.qkv_weight()
            qkv = F.linear(x, w, bias).view(b, length, 3, self.num_heads, self.head_dim)
            out = flash_spacetime_attention_qkv(qkv, feats, self.rel_proj.weight, self.rel_proj.bias, seqlens,
                                                None, *flags, key_padding_mask=key_padding_mask)
            return self.proj(out.reshape(b, length, -1))
        q, k, v = self.project_qkv(x, kv)
        out = flash_spacetime_attention(q, k, v, feats, self.rel_proj.weight, self.rel_proj.bias, seqlens,
                                        None, *flags, key_padding_mask=key_padding_mask)
        return self.proj(merge_heads(out))
