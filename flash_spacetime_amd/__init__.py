"""flash-spacetime for MI355X: spacetime-interval-biased attention on gfx950.

Drop-in for sevmag/flash-spacetime's package (src/flash_spacetime/
__init__.py): the same names are exported. Attention scores a pair by
`q . k + <q, R_ij>` with `R_ij = E(x_i, x_j) W^T + b`, where E sinusoidally
embeds the signed spacetime interval of two detector pulses; the fused
operators never build the `[B, L, L, C]` pair tensor. The operators run
hand-written HIP kernels through a C ABI (include/flash_spacetime.h) and are
imported lazily, so the package and its spec API import without a GPU.
"""

from .reference import (  # noqa: F401
    SINEMB_CLIP,
    SINEMB_INPUT_SCALE,
    SINEMB_N_FREQ,
    TIME_SCALE,
    attention_rel_oracle_inputs,
    float_padding_mask,
    merge_heads,
    pair_mask_bias,
    sinusoidal_frequencies,
    spacetime_attention_reference,
    spacetime_pair_features,
    split_heads,
    valid_row_mask,
)

__all__ = [
    "SpacetimeAttention",
    "flash_spacetime_attention",
    "flash_spacetime_attention_varlen",
    "flash_spacetime_attention_qkv",
    "flash_spacetime_forward",
    "flash_spacetime_backward",
    "spacetime_attention_reference",
    "spacetime_pair_features",
    "sinusoidal_frequencies",
    "attention_rel_oracle_inputs",
    "pair_mask_bias",
    "float_padding_mask",
    "valid_row_mask",
    "split_heads",
    "merge_heads",
    "TIME_SCALE",
    "SINEMB_INPUT_SCALE",
    "SINEMB_CLIP",
    "SINEMB_N_FREQ",
]

_OPS = {
    "SpacetimeAttention": "attention",
    "flash_spacetime_attention": "forward",
    "flash_spacetime_attention_varlen": "forward",
    "flash_spacetime_attention_qkv": "forward",
    "flash_spacetime_forward": "forward",
    "flash_spacetime_backward": "backward",
}


def __getattr__(name: str) -> object:
    """Import the operator modules on first use (reference __init__.py:57-68)."""
    if name in _OPS:
        import importlib

        return getattr(importlib.import_module(f".{_OPS[name]}", __name__), name)
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
