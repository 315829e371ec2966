"""GPU parity of the fused HIP forward against the CPU oracle.

Re-expresses the reference's forward contract (test_gpu.py:172-234):
finite output, padding rows exactly zero, the 2x-eager rule against the
float64 oracle, bitwise determinism; plus the BASELINE tolerances
(norm-relative error <= 1e-4 in fp32 without the embedding, <= 2e-2 in
bf16), both coordinate regimes (normalised and saturated detector units)
and the shapes of BASELINE configs 0-4 at reduced batch.
"""

import pytest
import torch

import oracle
from tests._cases import (
    FLAGS, assert_2x_rule, atol_for, eager_in_dtype, make_padded, rel_err, seed_of,
)

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from flash_spacetime_amd import (
        flash_spacetime_attention, flash_spacetime_forward,
    )

# (batch, length, heads, head_dim D, channels C). The first 13 are the
# reference's SHAPES (test_gpu.py:63-77, C == D) straddling the 16/32 tile
# edges; the rest are BASELINE's head layouts (D=32, C=16; D=C=64) and
# fp32/bf16 kernel variants with other (H, D, C).
SHAPES = [
    (2, 1, 4, 48, 48),
    (2, 3, 4, 48, 48),
    (2, 17, 4, 48, 48),
    (3, 32, 16, 48, 48),
    (2, 33, 16, 48, 48),
    (1, 64, 16, 48, 48),
    (2, 65, 1, 48, 48),
    (2, 127, 16, 48, 48),
    (2, 128, 4, 48, 48),
    (2, 200, 16, 48, 48),
    (1, 800, 16, 48, 48),
    (2, 33, 4, 16, 16),
    (2, 33, 4, 32, 32),
    (2, 96, 12, 32, 16),
    (3, 70, 12, 32, 16),
    (1, 150, 8, 64, 64),
    (2, 45, 6, 16, 64),
    (2, 50, 10, 64, 32),
]


def _to_gpu(case, dtype):
    dev = "cuda"
    return dict(
        q=case["q"].to(dev, dtype), k=case["k"].to(dev, dtype), v=case["v"].to(dev, dtype),
        feats=case["feats"].to(dev), weight=case["weight"].to(dev, dtype),
        bias=case["bias"].to(dev, dtype), seqlens=case["seqlens"].to(dev),
    )


def _fp64(case, flags):
    return oracle.attention_fp64_chunked(
        case["q"], case["k"], case["v"], case["feats"], case["weight"], case["bias"],
        case["seqlens"], use_attn_bias=flags[0], use_activation_bias=flags[1],
    )


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("flags", FLAGS, ids=lambda f: f"attn{int(f[0])}act{int(f[1])}")
@pytest.mark.parametrize("masked", [False, True], ids=["full", "masked"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_forward_matches_oracle(shape, flags, masked, dtype):
    case = make_padded(*shape, seed=seed_of("fwd", shape, flags, masked), masked=masked)
    g = _to_gpu(case, dtype)
    out, lse = flash_spacetime_forward(
        g["q"], g["k"], g["v"], g["feats"], g["weight"], g["bias"], g["seqlens"],
        use_attn_bias=flags[0], use_activation_bias=flags[1],
    )
    torch.cuda.synchronize()
    valid = oracle.valid_row_mask(shape[0], shape[1], case["seqlens"])
    assert out.dtype == dtype and out.shape == case["q"].shape
    assert torch.isfinite(out).all()
    pad = ~valid
    if pad.any():
        assert (out.permute(0, 2, 1, 3).cpu()[pad] == 0).all(), "padding rows must be exactly zero"
        assert (lse.permute(0, 2, 1).cpu()[pad] == 0).all()
    ref64, lse64 = _fp64(case, flags)
    vmask = valid[:, None, :, None].expand_as(ref64)
    eager = eager_in_dtype(case, flags, dtype)
    assert_2x_rule(out.cpu(), eager, ref64, vmask, atol_for(dtype, flags), "forward")
    # lse: the kernel drops the row-constant qt.b term of the logits.
    qt = case["q"] * shape[3] ** -0.5
    lse_ref = lse64 - (qt @ case["bias"] if flags[0] else 0.0)
    lmask = valid[:, None, :].expand_as(lse_ref)
    lse_tol = 1e-3 if dtype == torch.float32 else 5e-2
    torch.testing.assert_close(lse.double().cpu()[lmask], lse_ref[lmask], atol=lse_tol, rtol=lse_tol)
    # BASELINE relative tolerances.
    err = rel_err(out.cpu()[vmask], ref64[vmask])
    if dtype == torch.bfloat16:
        assert err <= 2e-2, f"bf16 relative error {err:.3e}"
    elif not (flags[0] or flags[1]):
        assert err <= 1e-4, f"fp32 relative error {err:.3e}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("shape", [(2, 96, 12, 32, 16), (2, 40, 8, 64, 64)],
                         ids=lambda s: "x".join(map(str, s)))
def test_forward_detector_units(shape, dtype):
    """Raw detector coordinates: every off-diagonal pair is saturated (x = +-4096)."""
    case = make_padded(*shape, seed=seed_of("det", shape), pos="detector")
    g = _to_gpu(case, dtype)
    out, _ = flash_spacetime_forward(g["q"], g["k"], g["v"], g["feats"], g["weight"], g["bias"],
                                     g["seqlens"])
    ref64, _ = _fp64(case, (True, True))
    valid = oracle.valid_row_mask(shape[0], shape[1], case["seqlens"])
    vmask = valid[:, None, :, None].expand_as(ref64)
    eager = eager_in_dtype(case, (True, True), dtype)
    assert_2x_rule(out.cpu(), eager, ref64, vmask, atol_for(dtype, (True, True)), "forward/detector")
    err = rel_err(out.cpu()[vmask], ref64[vmask])
    assert err <= (2e-2 if dtype == torch.bfloat16 else 1e-3), err


@pytest.mark.parametrize("shape", [(2, 17, 4, 48, 48), (2, 33, 16, 48, 48), (2, 200, 16, 48, 48),
                                   (2, 96, 12, 32, 16)], ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("flags", FLAGS[:2], ids=["attn1act1", "attn1act0"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_forward_deterministic(shape, flags, dtype):
    """Two identical calls give bitwise-identical output and LSE (test_gpu.py:211-234)."""
    case = make_padded(*shape, seed=1234)
    g = _to_gpu(case, dtype)
    args = (g["q"], g["k"], g["v"], g["feats"], g["weight"], g["bias"], g["seqlens"])
    out1, lse1 = flash_spacetime_forward(*args, use_attn_bias=flags[0], use_activation_bias=flags[1])
    out2, lse2 = flash_spacetime_forward(*args, use_attn_bias=flags[0], use_activation_bias=flags[1])
    assert torch.equal(out1, out2)
    assert torch.equal(lse1, lse2)


def test_mask_forms_agree():
    """seqlens, a bool padding mask and the float 0/-inf mask give one result."""
    shape = (3, 40, 4, 32, 16)
    case = make_padded(*shape, seed=77)
    g = _to_gpu(case, torch.bfloat16)
    valid = oracle.valid_row_mask(3, 40, case["seqlens"]).cuda()
    base = flash_spacetime_attention(g["q"], g["k"], g["v"], g["feats"], g["weight"], g["bias"],
                                     g["seqlens"])
    by_bool = flash_spacetime_attention(g["q"], g["k"], g["v"], g["feats"], g["weight"], g["bias"],
                                        key_padding_mask=~valid)
    by_float = flash_spacetime_attention(g["q"], g["k"], g["v"], g["feats"], g["weight"], g["bias"],
                                         oracle.float_padding_mask(valid, torch.float32))
    assert torch.equal(base, by_bool) and torch.equal(base, by_float)


def test_feats_requires_grad_raises():
    """Coordinates are detector data; a grad request must fail loud (test_gpu.py:327-340)."""
    case = make_padded(2, 17, 4, 48, 48, seed=5, masked=False)
    g = _to_gpu(case, torch.float32)
    feats = g["feats"].requires_grad_(True)
    with pytest.raises(ValueError, match="feats"):
        flash_spacetime_attention(g["q"], g["k"], g["v"], feats, g["weight"], g["bias"], g["seqlens"])


def test_unsupported_shapes_raise():
    case = make_padded(1, 8, 4, 32, 16, seed=6)
    g = _to_gpu(case, torch.float32)
    with pytest.raises(ValueError, match="C in"):
        flash_spacetime_forward(g["q"], g["k"], g["v"], g["feats"], g["weight"][:, :12], g["bias"],
                                g["seqlens"])
    # float64 is refused (float16 runs the bf16 path, tests/test_half_gpu.py)
    with pytest.raises(ValueError):
        flash_spacetime_forward(g["q"].double(), g["k"].double(), g["v"].double(), g["feats"], g["weight"],
                                g["bias"], g["seqlens"])
