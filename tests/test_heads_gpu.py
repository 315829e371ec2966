"""GPU tests of head counts the kernels do not take in one call.

More than 16 heads (and float32 at D = C = 64 with more than 8) run as the
fewest equal head groups the library has kernels for, each group's
operands copied to contiguous tensors, dW and db summed over the groups in
order. The reference pads heads to the next power of two inside one kernel
and takes any count (forward.py:22, backward.py:574). Checked against the
float64 oracle, and the grouped call bitwise against the same groups run
one by one through the public op, for padded, packed, token-major and
interleaved layouts.
"""

import pytest
import torch

import oracle
from tests._cases import make_padded, rel_err, seed_of

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from flash_spacetime_amd import (
        flash_spacetime_attention, flash_spacetime_attention_qkv, flash_spacetime_attention_varlen,
        flash_spacetime_backward, flash_spacetime_forward,
    )

DEV = "cuda"


@pytest.mark.parametrize("dtype,heads,dim,chans,tol", [
    (torch.bfloat16, 24, 32, 16, 2e-2),
    (torch.bfloat16, 17, 16, 32, 2e-2),
    (torch.float32, 12, 64, 64, 1e-4),
], ids=["bf16-h24", "bf16-h17", "fp32-h12-d64c64"])
def test_grouped_heads_match_oracle(dtype, heads, dim, chans, tol):
    case = make_padded(2, 70, heads, dim, chans, seed=seed_of("heads", heads, dim, chans), lens=[70, 29])
    gw = torch.randn(case["q"].shape, dtype=torch.float64, generator=torch.Generator().manual_seed(3))
    leaves = [case[n].to(DEV, dtype).requires_grad_(True) for n in ("q", "k", "v")]
    w = case["weight"].to(DEV, torch.float32).requires_grad_(True)
    b = case["bias"].to(DEV, torch.float32).requires_grad_(True)
    out = flash_spacetime_attention(*leaves, case["feats"].to(DEV), w, b, case["seqlens"].to(DEV))
    valid = oracle.valid_row_mask(2, 70, case["seqlens"]).to(DEV)[:, None, :, None]
    (out * gw.to(DEV, dtype) * valid).sum().backward()
    qr, kr, vr = (leaves[i].detach().double().cpu() for i in range(3))
    w64, b64 = w.detach().double().cpu(), b.detach().double().cpu()
    ref, _ = oracle.attention_fp64_chunked(qr, kr, vr, case["feats"], w64, b64, case["seqlens"])
    vm = valid.cpu().expand(ref.shape)
    assert rel_err(out.detach().double().cpu()[vm], ref[vm]) <= tol
    grads = oracle.backward_fp64_chunked(qr, kr, vr, case["feats"], w64, b64, gw * vm, case["seqlens"])
    for got, want, name in zip((leaves[0].grad, leaves[1].grad, leaves[2].grad, w.grad, b.grad), grads,
                               ("dq", "dk", "dv", "dW", "db")):
        err = rel_err(got.double().cpu(), want)
        assert err <= tol, f"{name}: {err:.3e}"


def _parts(t, groups):
    return [t[:, h0:h1].contiguous() for h0, h1 in groups]


def test_grouped_launchers_equal_groups_one_by_one():
    heads, groups = 20, [(0, 10), (10, 20)]
    case = make_padded(3, 90, heads, 32, 16, seed=seed_of("heads-split"), pos="detector")
    q, k, v = (case[n].to(DEV, torch.bfloat16) for n in ("q", "k", "v"))
    do = torch.randn(q.shape, generator=torch.Generator().manual_seed(5)).to(DEV, torch.bfloat16)
    feats, sl = case["feats"].to(DEV), case["seqlens"].to(DEV)
    w, b = case["weight"].to(DEV, torch.float32), case["bias"].to(DEV, torch.float32)
    out, lse = flash_spacetime_forward(q, k, v, feats, w, b, sl)
    rowsum = torch.empty_like(lse)
    dq, dk, dv, dw, db = flash_spacetime_backward(q, k, v, feats, w, b, sl, lse, do, rowsum=rowsum)
    dw_sum = torch.zeros_like(dw)
    db_sum = torch.zeros_like(db)
    for (h0, h1), qg, kg, vg, dog in zip(groups, _parts(q, groups), _parts(k, groups), _parts(v, groups),
                                         _parts(do, groups)):
        og, lg = flash_spacetime_forward(qg, kg, vg, feats, w, b, sl)
        rg = torch.empty_like(lg)
        gq, gk, gv, gw, gb = flash_spacetime_backward(qg, kg, vg, feats, w, b, sl, lg, dog, rowsum=rg)
        assert torch.equal(out[:, h0:h1], og) and torch.equal(lse[:, h0:h1], lg)
        assert torch.equal(rowsum[:, h0:h1], rg)
        for full, part in ((dq, gq), (dk, gk), (dv, gv)):
            assert torch.equal(full[:, h0:h1], part)
        dw_sum += gw
        db_sum += gb
    assert torch.equal(dw, dw_sum) and torch.equal(db, db_sum)


def _step(fn, leaves, do):
    out = fn(*leaves)
    out.backward(do)
    return out.detach(), [x.grad for x in leaves]


def test_grouped_layouts_equal_contiguous_op():
    """Token-major views and the interleaved QKV op with 20 heads give the
    contiguous padded op's results bitwise; packed events give those of
    their head groups run one by one."""
    gen = torch.Generator().manual_seed(17)
    batch, length, heads, dim = 2, 64, 20, 16
    lens = torch.tensor([64, 23], dtype=torch.int32, device=DEV)
    qkv = torch.randn(batch, length, 3, heads, dim, generator=gen).to(DEV, torch.bfloat16)
    feats = torch.cat([(torch.rand(batch, length, 3, generator=gen) - 0.5) * 1000,
                       torch.rand(batch, length, 1, generator=gen) * 2e4], -1).to(DEV)
    w = (torch.randn(dim, 16, generator=gen) / 4).to(DEV)
    b = (torch.randn(dim, generator=gen) * 0.02).to(DEV)
    do = torch.randn(batch, heads, length, dim, generator=gen).to(DEV, torch.bfloat16)
    # reference: contiguous [B, H, L, D] operands
    base = [qkv[:, :, i].transpose(1, 2).contiguous().requires_grad_(True) for i in range(3)]
    ref_out, ref_grads = _step(lambda q, k, v: flash_spacetime_attention(q, k, v, feats, w, b, lens), base, do)
    # token-major views of [B, L, H, D]
    tm = [qkv[:, :, i].contiguous().transpose(1, 2).requires_grad_(True) for i in range(3)]
    out, grads = _step(lambda q, k, v: flash_spacetime_attention(q, k, v, feats, w, b, lens), tm, do)
    assert torch.equal(out, ref_out) and all(torch.equal(g, r) for g, r in zip(grads, ref_grads))
    # the fused QKV op: [B, L, 3, H, D] in, [B, L, H, D] out
    leaf = qkv.clone().requires_grad_(True)
    out = flash_spacetime_attention_qkv(leaf, feats, w, b, lens)
    out.backward(do.transpose(1, 2))
    assert torch.equal(out.transpose(1, 2), ref_out)
    for i in range(3):
        assert torch.equal(leaf.grad[:, :, i].transpose(1, 2), ref_grads[i])
    # packed events: the grouped call against its two head groups run one by one
    cu = torch.tensor([0, 64, 87], dtype=torch.int32, device=DEV)
    pk = lambda t, n: t[n, :, :int(lens[n])].transpose(0, 1)  # noqa: E731
    packed = [torch.cat([pk(x.detach(), 0), pk(x.detach(), 1)]).requires_grad_(True) for x in base]
    pfeats = torch.cat([feats[0, :64], feats[1, :23]])
    pdo = torch.cat([pk(do, 0), pk(do, 1)])
    varlen = lambda q, k, v: flash_spacetime_attention_varlen(q, k, v, pfeats, w, b, cu)  # noqa: E731
    out, grads = _step(varlen, packed, pdo)
    for h0, h1 in ((0, 10), (10, 20)):
        part = [x.detach()[:, h0:h1].contiguous().requires_grad_(True) for x in packed]
        o, g = _step(varlen, part, pdo[:, h0:h1].contiguous())
        assert torch.equal(out[:, h0:h1], o)
        assert all(torch.equal(a[:, h0:h1], c) for a, c in zip(grads, g))
