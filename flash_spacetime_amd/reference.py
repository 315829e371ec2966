"""Specification-side API of flash-spacetime (pure PyTorch, any device).

Same names, constants and semantics as the reference module
(src/flash_spacetime/reference.py), generalised from `W [C, C], C == D` to
the nn.Linear layout `W [D, C]`. These functions define the operation; the
fused operators in `flash_spacetime_amd.forward` never call them (they run
the HIP kernels or raise) -- they exist so code written against the
reference's spec API keeps working, e.g. for A/B checks against the
materialised definition on small inputs.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import Tensor

# reference.py:39-42 (3e4 / 500 * 3e-1 is exactly 18.0)
TIME_SCALE = 3e4 / 500 * 3e-1
SINEMB_INPUT_SCALE = 1024.0
SINEMB_CLIP = 4.0
SINEMB_N_FREQ = 10000.0


def sinusoidal_frequencies(dim: int, device: torch.device) -> Tensor:
    """fp32 ladder `exp(-i ln(1e4) / (dim/2))`, i < dim/2 (reference.py:45-56)."""
    half = dim / 2
    step = -(torch.log(torch.tensor([SINEMB_N_FREQ], device=device)) / half)
    return torch.exp(torch.arange(half, device=device) * step)


def spacetime_pair_features(feats: Tensor, weight: Tensor, bias: Optional[Tensor]) -> Tensor:
    """`R_ij = W E_ij + b`, `[B, L, L, D]`; weight `[D, C]` (reference.py:59-88).

    E_ij holds sin then cos of `x_ij * f` with
    `x_ij = 1024 clip(sign(I) sqrt|I|, -4, 4)` and
    `I = |p_i - p_j|^2 - (18 (t_i - t_j))^2` (positions in feats columns 0-2,
    the interval's time in column 3). The embedding is cast to the weight
    dtype before the projection.
    """
    xyz, tcol = feats[:, :, :3], feats[:, :, 3]
    interval = (xyz[:, :, None] - xyz[:, None, :]).pow(2).sum(-1) - (
        (tcol[:, :, None] - tcol[:, None, :]) * TIME_SCALE
    ).pow(2)
    signed = torch.sign(interval) * torch.sqrt(torch.abs(interval))
    x = SINEMB_INPUT_SCALE * signed.clip(-SINEMB_CLIP, SINEMB_CLIP)
    theta = x.unsqueeze(-1) * sinusoidal_frequencies(weight.shape[1], feats.device)
    emb = torch.cat((torch.sin(theta), torch.cos(theta)), dim=-1)
    return torch.nn.functional.linear(emb.to(weight.dtype), weight, bias)


def pair_mask_bias(key_padding_mask: Tensor) -> Tensor:
    """`[B, L, L]` -inf where exactly one token of the pair is padding (reference.py:91-103)."""
    row, col = key_padding_mask[:, :, None], key_padding_mask[:, None, :]
    out = torch.minimum(row, col).clone()
    out[torch.maximum(row, col) < 0] = 0
    return out


def spacetime_attention_reference(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    feats: Tensor,
    weight: Tensor,
    bias: Optional[Tensor],
    key_padding_mask: Optional[Tensor] = None,
    scale: Optional[float] = None,
    use_attn_bias: bool = True,
    use_activation_bias: bool = True,
) -> Tensor:
    """Materialised definition of the op (reference.py:106-167), weight `[D, C]`."""
    head_dim = q.shape[-1]
    if weight.shape[0] != head_dim:
        raise ValueError(f"weight must be [D={head_dim}, C], got {tuple(weight.shape)}")
    qt = q * (head_dim ** -0.5 if scale is None else scale)
    logits = qt @ k.transpose(-2, -1)
    rel = None
    if use_attn_bias or use_activation_bias:
        rel = spacetime_pair_features(feats, weight, bias)
    if use_attn_bias:
        logits = logits + torch.einsum("bhid,bijd->bhij", qt, rel)
    if key_padding_mask is not None:
        logits = logits + pair_mask_bias(key_padding_mask).unsqueeze(1)
    probs = logits.softmax(dim=-1)
    out = probs.to(v.dtype) @ v
    if use_activation_bias:
        out = out + torch.einsum("bhij,bijd->bhid", probs.to(rel.dtype), rel)
    return out


def valid_row_mask(batch_size: int, length: int, seqlens: Tensor) -> Tensor:
    """`[B, L]` True on the first `seqlens[b]` tokens (reference.py:170-177)."""
    return torch.arange(length, device=seqlens.device)[None, :] < seqlens[:, None]


def float_padding_mask(valid: Tensor, dtype: torch.dtype) -> Tensor:
    """0 on valid tokens, -inf on padding (reference.py:180-184)."""
    out = torch.zeros(valid.shape, dtype=dtype, device=valid.device)
    out.masked_fill_(~valid, float("-inf"))
    return out


def split_heads(x: Tensor, num_heads: int) -> Tensor:
    """`[B, L, H*D]` -> `[B, H, L, D]` (reference.py:187-190)."""
    b, length, _ = x.shape
    return x.reshape(b, length, num_heads, -1).permute(0, 2, 1, 3)


def merge_heads(x: Tensor) -> Tensor:
    """`[B, H, L, D]` -> `[B, L, H*D]` (reference.py:193-195)."""
    return x.transpose(1, 2).reshape(x.shape[0], x.shape[2], -1)


def attention_rel_oracle_inputs(
    attention: torch.nn.Module, x: Tensor, kv: Optional[Tensor] = None
) -> Tuple[Tensor, Tensor, Tensor]:
    """Per-head q, k, v as graphnet's `Attention_rel.forward` builds them (reference.py:198-223)."""
    kv = x if kv is None else kv
    q = torch.nn.functional.linear(x, attention.proj_q.weight, attention.q_bias)
    k = torch.nn.functional.linear(kv, attention.proj_k.weight, None)
    v = torch.nn.functional.linear(kv, attention.proj_v.weight, attention.v_bias)
    h = attention.num_heads
    return split_heads(q, h), split_heads(k, h), split_heads(v, h)
