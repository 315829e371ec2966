"""Seeded inputs and comparison rules shared by the GPU parity tests.

Inputs are drawn on the CPU from one seeded generator in float64 (as the
reference's tests do, test_gpu.py:81-108, test_varlen.py:47-73) and cast per
test. Expected values come from the CPU oracle (`oracle/`): the float64
chunked evaluators are the truth, the eager restatement in the test dtype is
the "eager error" yardstick of the reference's 2x-eager rule
(test_gpu.py:133-169).
"""

from __future__ import annotations

import zlib
from typing import Dict, Optional, Sequence, Tuple

import torch

import oracle

ATOL = {torch.float32: 1e-6, torch.bfloat16: 1e-2}
ATOL_FP32_WITH_E = 5e-3
ULP = {torch.bfloat16: 2.0 ** -8, torch.float32: 2.0 ** -23}
FLAGS = [(True, True), (True, False), (False, True), (False, False)]


def seed_of(*key) -> int:
    """Process-independent seed (the reference's hash() seeds vary per process)."""
    return zlib.crc32(repr(key).encode()) & 0x7FFFFFFF


def atol_for(dtype: torch.dtype, flags: Tuple[bool, bool]) -> float:
    if dtype is torch.float32 and (flags[0] or flags[1]):
        return ATOL_FP32_WITH_E
    return ATOL[dtype]


def make_padded(batch: int, length: int, heads: int, dim: int, channels: int, seed: int,
                masked: bool = True, pos: str = "normal", lens: Optional[Sequence[int]] = None,
                qk_scale: float = 1.0) -> Dict[str, torch.Tensor]:
    """Padded case on the CPU in float64. pos: 'normal' (randn features, the
    reference tests' distribution) or 'detector' (x,y,z ~ U(-500,500),
    t ~ U(0,2e4): every off-diagonal pair saturates the clip)."""
    gen = torch.Generator().manual_seed(seed)

    def rn(*shape):
        return torch.randn(*shape, generator=gen, dtype=torch.float64)

    case = {
        "q": rn(batch, heads, length, dim) * qk_scale,
        "k": rn(batch, heads, length, dim) * qk_scale,
        "v": rn(batch, heads, length, dim),
    }
    if pos == "normal":
        case["feats"] = rn(batch, length, 5)
    else:
        xyz = (torch.rand(batch, length, 3, generator=gen, dtype=torch.float64) - 0.5) * 1000
        t = torch.rand(batch, length, 1, generator=gen, dtype=torch.float64) * 2e4
        case["feats"] = torch.cat([xyz, t, rn(batch, length, 1)], -1)
    case["weight"] = rn(dim, channels) / channels ** 0.5
    case["bias"] = rn(dim)
    if lens is not None:
        seqlens = torch.tensor(list(lens), dtype=torch.long)
    elif masked and length > 1:
        seqlens = torch.randint(1, length + 1, (batch,), generator=gen)
        seqlens[0] = length
        if batch > 1:
            seqlens[-1] = 1
    else:
        seqlens = torch.full((batch,), length, dtype=torch.long)
    case["seqlens"] = seqlens
    return case


def make_packed(lengths: Sequence[int], heads: int, dim: int, channels: int, seed: int,
                pos: str = "normal") -> Dict[str, torch.Tensor]:
    gen = torch.Generator().manual_seed(seed)
    total = int(sum(lengths))

    def rn(*shape):
        return torch.randn(*shape, generator=gen, dtype=torch.float64)

    case = {"q": rn(total, heads, dim), "k": rn(total, heads, dim), "v": rn(total, heads, dim)}
    if pos == "normal":
        case["feats"] = rn(total, 5)
    else:
        xyz = (torch.rand(total, 3, generator=gen, dtype=torch.float64) - 0.5) * 1000
        t = torch.rand(total, 1, generator=gen, dtype=torch.float64) * 2e4
        case["feats"] = torch.cat([xyz, t], -1)
    case["weight"] = rn(dim, channels) / channels ** 0.5
    case["bias"] = rn(dim)
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + int(n))
    case["cu"] = torch.tensor(cu, dtype=torch.int32)
    return case


def eager_in_dtype(case, flags, dtype) -> torch.Tensor:
    """The eager definition evaluated in the test dtype (reference test_gpu.py:111-130)."""
    valid = oracle.valid_row_mask(case["q"].shape[0], case["q"].shape[2], case["seqlens"])
    mask = oracle.float_padding_mask(valid, torch.float32)
    fdt = torch.float64 if dtype == torch.float64 else torch.float32
    return oracle.attention(
        case["q"].to(dtype), case["k"].to(dtype), case["v"].to(dtype), case["feats"].to(fdt),
        case["weight"].to(dtype), case["bias"].to(dtype), key_padding_mask=mask,
        use_attn_bias=flags[0], use_activation_bias=flags[1],
    )


def assert_2x_rule(kernel_out, dtype_ref, fp64_ref, valid, atol, what, reduction=False):
    """|kernel - ref64| <= 2 |eager - ref64| + atol + 8 ulp max(|ref64|, 1), and
    mean(kernel_err) <= 1.5 mean(eager_err) + atol (reference test_gpu.py:133-169)."""
    kernel_err = (kernel_out.double().cpu() - fp64_ref)[valid].abs()
    eager_err = (dtype_ref.double().cpu() - fp64_ref)[valid].abs()
    if kernel_err.numel() == 0:
        return
    ulp = ULP.get(kernel_out.dtype, 0.0)
    floor = atol + 8.0 * ulp * fp64_ref[valid].abs().clamp(min=1.0)
    ref_err = torch.maximum(eager_err, eager_err.median()) if reduction else eager_err
    bound = 2.0 * ref_err + floor
    bad = kernel_err > bound
    assert not bad.any(), (
        f"{what}: {int(bad.sum())} elements exceed the 2x-eager bound; worst kernel err "
        f"{kernel_err.max():.3e} vs bound {bound[kernel_err.argmax()]:.3e}"
    )
    assert kernel_err.mean() <= 1.5 * eager_err.mean() + atol, (
        f"{what}: kernel mean error {kernel_err.mean():.3e} exceeds 1.5x eager mean "
        f"{eager_err.mean():.3e}"
    )


def rel_err(got: torch.Tensor, want: torch.Tensor) -> float:
    """Norm-relative error ||got - want|| / ||want||."""
    g = got.double().cpu()
    w = want.double().cpu()
    den = w.norm().item()
    return (g - w).norm().item() / (den if den > 0 else 1.0)
