"""The bf16 rows kernel with a reference D from the forward's output.

Given the forward's output, the rows kernel forms dS = P (dP - D_ref) with
D_ref = dO . (out - b) (b with the activation bias), and corrects its sums
to its own D = sum P dP / sum P once, after its last key chunk:
dQ -= (D - D_ref) sum P k, H -= (D - D_ref) G. Without it, D is formed
online and the sums are corrected after every chunk. Both hold the same D
(so rowsum(dS) = 0 the same way), so the gradients agree up to rounding:
each path is held to the float64 oracle on the bf16-rounded inputs, also
where the values carry a large common offset (|D| much larger than the
spread of dP, where the rounding of dS depends most on the D it is formed
against). The autograd op hands its output to the backward unless the
output was modified in place since.
"""

import pytest
import torch

import oracle
from tests._cases import make_packed, make_padded, rel_err, seed_of

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from flash_spacetime_amd import (
        flash_spacetime_attention, flash_spacetime_attention_varlen, flash_spacetime_backward,
        flash_spacetime_forward,
    )

DEV = "cuda"
BF = torch.bfloat16
FLAGS = [(True, True), (True, False), (False, True)]
SHAPES = [(2, 96, 12, 32, 16), (3, 160, 12, 32, 16), (1, 130, 8, 64, 64), (2, 70, 16, 48, 32),
          (2, 33, 4, 16, 16)]


def _padded(case, flags, v_offset):
    """Both backward paths and the float64 oracle's gradients on one padded case."""
    for key in ("q", "k"):
        case[key] = case[key].to(BF).double()
    case["v"] = (case["v"] + v_offset).to(BF).double()
    q, k, v = (case[x].to(DEV, BF) for x in ("q", "k", "v"))
    feats, sl = case["feats"].to(DEV), case["seqlens"].to(DEV)
    w, b = case["weight"].float().to(DEV), case["bias"].float().to(DEV)
    kw = dict(use_attn_bias=flags[0], use_activation_bias=flags[1])
    out, lse = flash_spacetime_forward(q, k, v, feats, w, b, sl, **kw)
    do = torch.randn(q.shape, generator=torch.Generator().manual_seed(3)).to(BF)
    online = flash_spacetime_backward(q, k, v, feats, w, b, sl, lse, do.to(DEV), **kw)
    refd = flash_spacetime_backward(q, k, v, feats, w, b, sl, lse, do.to(DEV), out=out, **kw)
    valid = oracle.valid_row_mask(q.shape[0], q.shape[2], case["seqlens"])[:, None, :, None]
    ref = oracle.backward_fp64_chunked(case["q"], case["k"], case["v"], case["feats"], w.double().cpu(),
                                       b.double().cpu(), do.double() * valid, case["seqlens"], **kw)
    return online, refd, ref


def _check(online, refd, ref, flags, what):
    for name, a, r, e in zip(("dq", "dk", "dv", "dW", "db"), online, refd, ref):
        if name == "db" and not flags[1]:
            continue
        ea, er = rel_err(a.cpu(), e), rel_err(r.cpu(), e)
        print(f"{what} {name}: online {ea:.2e} reference-D {er:.2e} apart {rel_err(r.cpu(), a.cpu()):.2e}",
              flush=True)
        assert ea <= 2e-2 and er <= 2e-2, (name, ea, er)


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("flags", FLAGS, ids=["attn1act1", "attn1act0", "attn0act1"])
@pytest.mark.parametrize("v_offset", [0.0, 6.0], ids=["centred", "offset"])
def test_reference_d_matches_oracle(shape, flags, v_offset):
    case = make_padded(*shape, seed=seed_of("refd", shape, flags, v_offset))
    online, refd, ref = _padded(case, flags, v_offset)
    _check(online, refd, ref, flags, f"{shape} {flags} offset {v_offset}")


@pytest.mark.parametrize("pos", ["normal", "detector"])
def test_reference_d_packed(pos):
    """Packed events of mixed lengths (many tiles, one tile, one token).
    (Peaked rows, q and k x30, are held by the self-consistency tests: there
    dq is zero in exact arithmetic and a relative error says nothing.)"""
    lens = [200, 17, 1, 64, 33]
    case = make_packed(lens, 12, 32, 16, seed=seed_of("refd-packed", pos), pos=pos)
    for key in ("q", "k"):
        case[key] = case[key].to(BF).double()
    case["v"] = case["v"].to(BF).double()
    q, k, v = (case[x].to(DEV, BF) for x in ("q", "k", "v"))
    feats, cu = case["feats"].to(DEV), case["cu"].to(DEV)
    w, b = case["weight"].float().to(DEV), case["bias"].float().to(DEV)
    out, lse = flash_spacetime_forward(q, k, v, feats, w, b, None, cu_seqlens=cu)
    do = torch.randn(q.shape, generator=torch.Generator().manual_seed(4)).to(BF)
    online = flash_spacetime_backward(q, k, v, feats, w, b, None, lse, do.to(DEV), cu_seqlens=cu)
    refd = flash_spacetime_backward(q, k, v, feats, w, b, None, lse, do.to(DEV), cu_seqlens=cu, out=out)
    ref = oracle.backward_fp64_chunked(case["q"], case["k"], case["v"], case["feats"], w.double().cpu(),
                                       b.double().cpu(), do.double(), None, cu_seqlens=case["cu"])
    _check(online, refd, ref, (True, True), f"packed {pos}")


def test_reference_d_deterministic():
    case = make_padded(3, 150, 12, 32, 16, seed=98)
    q, k, v = (case[x].to(DEV, BF) for x in ("q", "k", "v"))
    feats, sl = case["feats"].to(DEV), case["seqlens"].to(DEV)
    w, b = case["weight"].float().to(DEV), case["bias"].float().to(DEV)
    out, lse = flash_spacetime_forward(q, k, v, feats, w, b, sl)
    do = torch.randn(q.shape, generator=torch.Generator().manual_seed(5)).to(DEV, BF)
    r1 = flash_spacetime_backward(q, k, v, feats, w, b, sl, lse, do, out=out)
    r2 = flash_spacetime_backward(q, k, v, feats, w, b, sl, lse, do, out=out)
    for a, c in zip(r1, r2):
        assert torch.equal(a, c)


def _leaves(case):
    return [case[x].to(DEV, BF).requires_grad_(True) for x in ("q", "k", "v")]


def test_autograd_hands_over_its_output():
    """The op's backward runs the reference-D path with its own output (bit
    for bit the direct call with out=), and the online path once the output
    was modified in place (bit for bit the direct call without it)."""
    case = make_padded(2, 96, 12, 32, 16, seed=97)
    feats, sl = case["feats"].to(DEV), case["seqlens"].to(DEV)
    w, b = case["weight"].float().to(DEV), case["bias"].float().to(DEV)
    do = torch.randn(case["q"].shape, generator=torch.Generator().manual_seed(6)).to(DEV, BF)
    q, k, v = (case[x].to(DEV, BF) for x in ("q", "k", "v"))
    out, lse = flash_spacetime_forward(q, k, v, feats, w, b, sl)
    with_out = flash_spacetime_backward(q, k, v, feats, w, b, sl, lse, do, out=out)
    without = flash_spacetime_backward(q, k, v, feats, w, b, sl, lse, 2 * do)

    leaves = _leaves(case)
    o = flash_spacetime_attention(*leaves, feats, w, b, sl)
    assert torch.equal(o.detach(), out)
    o.backward(do)
    for leaf, g in zip(leaves, with_out[:3]):
        assert torch.equal(leaf.grad, g)

    leaves = _leaves(case)
    o = flash_spacetime_attention(*leaves, feats, w, b, sl)
    o.mul_(2.0)  # the kept output no longer matches what the forward returned
    o.backward(do)
    for leaf, g in zip(leaves, without[:3]):
        assert torch.equal(leaf.grad, g)


def test_varlen_autograd_reference_d():
    """The packed op through autograd (reference-D path) against the oracle."""
    lens = [90, 5, 40]
    case = make_packed(lens, 8, 32, 16, seed=96)
    for key in ("q", "k", "v"):
        case[key] = case[key].to(BF).double()
    leaves = [case[x].to(DEV, BF).requires_grad_(True) for x in ("q", "k", "v")]
    w, b = case["weight"].float().to(DEV), case["bias"].float().to(DEV)
    cu = case["cu"].to(DEV)
    o = flash_spacetime_attention_varlen(*leaves, case["feats"].to(DEV), w, b, cu)
    do = torch.randn(o.shape, generator=torch.Generator().manual_seed(7)).to(DEV, BF)
    o.backward(do)
    ref = oracle.backward_fp64_chunked(case["q"], case["k"], case["v"], case["feats"], w.double().cpu(),
                                       b.double().cpu(), do.double().cpu(), None, cu_seqlens=case["cu"])
    for leaf, e in zip(leaves, ref[:3]):
        assert rel_err(leaf.grad.cpu(), e) <= 2e-2


def test_nonfinite_output_is_not_used():
    """An output with non-finite values (not this forward's) is not a usable
    reference: the kernel falls back to 0 for it, and the gradients stay
    finite and within the bf16 tolerance of the float64 ones."""
    case = make_padded(2, 96, 12, 32, 16, seed=95)
    for key in ("q", "k", "v"):
        case[key] = case[key].to(BF).double()
    q, k, v = (case[x].to(DEV, BF) for x in ("q", "k", "v"))
    feats, sl = case["feats"].to(DEV), case["seqlens"].to(DEV)
    w, b = case["weight"].float().to(DEV), case["bias"].float().to(DEV)
    out, lse = flash_spacetime_forward(q, k, v, feats, w, b, sl)
    do = torch.randn(q.shape, generator=torch.Generator().manual_seed(8)).to(BF)
    bad = torch.full_like(out, float("nan"))
    bad[:, :, 1::2] = float("inf")
    got = flash_spacetime_backward(q, k, v, feats, w, b, sl, lse, do.to(DEV), out=bad)
    valid = oracle.valid_row_mask(q.shape[0], q.shape[2], case["seqlens"])[:, None, :, None]
    ref = oracle.backward_fp64_chunked(case["q"], case["k"], case["v"], case["feats"], w.double().cpu(),
                                       b.double().cpu(), do.double() * valid, case["seqlens"])
    for name, a, e in zip(("dq", "dk", "dv", "dW", "db"), got, ref):
        assert torch.isfinite(a).all(), name
        assert rel_err(a.cpu(), e) <= 2e-2, name


def test_kept_output_goes_through_saved_tensor_hooks():
    """The output the backward keeps is a saved tensor like the inputs:
    saved-tensor hooks (here counting and offloading, as save_on_cpu does)
    see it, and the gradients are bit for bit those of the plain run. The
    float16 op, whose result is converted from a temporary bf16 output, keeps
    nothing of it."""
    case = make_padded(2, 80, 12, 32, 16, seed=98)
    feats, sl = case["feats"].to(DEV), case["seqlens"].to(DEV)
    w, b = case["weight"].float().to(DEV), case["bias"].float().to(DEV)
    do = torch.randn(case["q"].shape, generator=torch.Generator().manual_seed(8)).to(DEV, BF)

    leaves = _leaves(case)
    flash_spacetime_attention(*leaves, feats, w, b, sl).backward(do)
    plain = [x.grad for x in leaves]

    packed = []

    def pack(t):
        packed.append((tuple(t.shape), t.dtype))
        return t.to("cpu")

    def unpack(t):
        return t.to(DEV)

    leaves = _leaves(case)
    with torch.autograd.graph.saved_tensors_hooks(pack, unpack):
        o = flash_spacetime_attention(*leaves, feats, w, b, sl)
    o.backward(do)
    assert (tuple(o.shape), BF) in packed[6:], packed  # after q, k, v, pos, lengths, lse
    for leaf, g in zip(leaves, plain):
        assert torch.equal(leaf.grad, g)

    packed.clear()
    half = [case[x].to(DEV, torch.float16).requires_grad_(True) for x in ("q", "k", "v")]
    with torch.autograd.graph.saved_tensors_hooks(pack, unpack):
        o = flash_spacetime_attention(*half, feats, w, b, sl)
    o.backward(do.to(torch.float16))
    assert not any(s == tuple(o.shape) and d == BF for s, d in packed[6:]), packed
