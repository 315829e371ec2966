"""GPU parity of the model-side module against the float64 oracle.

`SpacetimeAttention` (fused QKV GEMM read in place by the op, output
projection; cross-attention through three linears) against the composition
the reference's caller performs, built from the oracle on the CPU in
float64: `attention_rel_oracle_inputs` (reference.py:198-223), the eager
spec with the one-sided key mask, `merge_heads`, `proj`. Valid rows only
(padding rows of the module's output are `proj(0)`). Output and the
gradients of x and every parameter.
"""

import copy

import pytest
import torch

import oracle
from tests._cases import rel_err, seed_of

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from flash_spacetime_amd import SpacetimeAttention, attention_rel_oracle_inputs, merge_heads


def _holey(batch, length, gen):
    valid = torch.rand(batch, length, generator=gen) < 0.7
    valid[:, 0] = True
    return valid


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("qkv_bias", [False, True], ids=["nobias", "qkvbias"])
@pytest.mark.parametrize("mask", ["lengths", "holes", "cross"])
def test_module_matches_oracle_composition(dtype, qkv_bias, mask):
    batch, length, heads, dim = 3, 48, 4, 128  # head_dim 32
    gen = torch.Generator().manual_seed(seed_of("model", dtype, qkv_bias, mask))
    ref = SpacetimeAttention(dim, heads, channels=16, qkv_bias=qkv_bias, dtype=torch.float64)
    with torch.no_grad():
        for p in ref.parameters():
            p.copy_(torch.randn(p.shape, generator=gen, dtype=torch.float64) * (p.shape[-1] ** -0.5))
    # The module in the test dtype; the oracle runs on its rounded parameters.
    mod = copy.deepcopy(ref).to("cuda", dtype)
    with torch.no_grad():
        for p, r in zip(mod.parameters(), ref.parameters()):
            r.copy_(p.double().cpu())
    x64 = torch.randn(batch, length, dim, generator=gen, dtype=torch.float64).to(dtype).double()
    feats = torch.randn(batch, length, 5, generator=gen, dtype=torch.float64)
    kv64 = None
    if mask == "cross":
        kv64 = torch.randn(batch, length, dim, generator=gen, dtype=torch.float64).to(dtype).double()
    if mask in ("lengths", "cross"):
        lens = torch.tensor([length, 17, 1])
        valid = torch.arange(length)[None, :] < lens[:, None]
        kwargs = {"seqlens": lens.to("cuda")}
    else:
        valid = _holey(batch, length, gen)
        kwargs = {"key_padding_mask": (~valid).to("cuda")}
    gw = torch.randn(batch, length, dim, generator=gen, dtype=torch.float64) * valid[..., None]

    x = x64.to("cuda", dtype).requires_grad_(True)
    kv = None if kv64 is None else kv64.to("cuda", dtype)
    out = mod(x, feats.to("cuda"), kv=kv, **kwargs)
    (out.double() * gw.to("cuda")).sum().backward()

    xr = x64.clone().requires_grad_(True)
    q, k, v = attention_rel_oracle_inputs(ref, xr, kv64)
    att = oracle.attention(q, k, v, feats, ref.rel_proj.weight, ref.rel_proj.bias,
                           key_padding_mask=oracle.float_padding_mask(valid, torch.float64))
    want = ref.proj(merge_heads(att))
    (want * gw).sum().backward()

    vm = valid[..., None].expand(want.shape)
    # fp32: the op's own bound is 1e-4 (its error comes from evaluating the
    # embedding's sin / cos at arguments up to 4096 rad in fp32); the output
    # projection mixes H*D channels whose errors are independent, which moves
    # the relative error of the composition by a small factor either way.
    tol = 2e-2 if dtype == torch.bfloat16 else 2e-4
    gtol = 2e-2 if dtype == torch.bfloat16 else 1e-3
    err = rel_err(out.detach().double().cpu() * vm, want.detach() * vm)
    assert err <= tol, f"output: relative error {err:.3e}"
    err = rel_err(x.grad.double().cpu(), xr.grad)
    assert err <= gtol, f"grad x: relative error {err:.3e}"
    for (name, p), r in zip(mod.named_parameters(), ref.parameters()):
        assert p.grad is not None, name
        err = rel_err(p.grad.double().cpu(), r.grad)
        assert err <= gtol, f"grad {name}: relative error {err:.3e}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_module_packed_matches_padded(dtype):
    """Packed events (x [T, dim], cu_seqlens) through the module give the
    valid rows of the padded call on the same events, and the same input and
    parameter gradients (to tolerances: the GEMMs run on differently shaped
    operands)."""
    lens = [17, 1, 40, 9]
    batch, length, heads, dim = len(lens), max(lens), 4, 128
    gen = torch.Generator().manual_seed(seed_of("model-packed", dtype))
    mod = SpacetimeAttention(dim, heads, channels=16, qkv_bias=True, device="cuda", dtype=dtype)
    with torch.no_grad():
        for p in mod.parameters():
            p.copy_(torch.randn(p.shape, generator=gen).to(p) * (p.shape[-1] ** -0.5))
    xp = torch.randn(batch, length, dim, generator=gen).to("cuda", dtype)
    fp = torch.randn(batch, length, 4, generator=gen).to("cuda")
    valid = torch.arange(length)[None, :] < torch.tensor(lens)[:, None]
    gy = torch.randn(batch, length, dim, generator=gen).to("cuda", dtype) * valid[..., None].to("cuda", dtype)

    x1 = xp.clone().requires_grad_(True)
    out1 = mod(x1, fp, torch.tensor(lens, device="cuda"))
    (out1.float() * gy.float()).sum().backward()
    g1 = [p.grad.clone() for p in mod.parameters()]
    mod.zero_grad()

    vd = valid.to("cuda")
    x2 = xp[vd].clone().requires_grad_(True)
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32, device="cuda")
    out2 = mod(x2, fp[vd], cu_seqlens=cu)
    (out2.float() * gy[vd].float()).sum().backward()
    tol = 2e-2 if dtype == torch.bfloat16 else 1e-5
    assert rel_err(out2.detach().double().cpu(), out1.detach()[vd].double().cpu()) <= tol
    assert rel_err(x2.grad.double().cpu(), x1.grad[vd].double().cpu()) <= tol
    for a, p in zip(g1, mod.parameters()):
        assert rel_err(p.grad.double().cpu(), a.double().cpu()) <= tol
