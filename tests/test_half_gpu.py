"""GPU tests of float16 operands.

The reference computes every operand that is not float32 in bf16
(forward.py:271, backward.py:523), so float16 inputs run the bf16 kernels
here too and results come back in float16: the same values as the bf16 op
on the inputs rounded to bf16, cast to float16, and within the bf16
tolerance of the float64 oracle.
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


def test_half_padded_op_runs_the_bf16_path():
    case = make_padded(2, 60, 6, 32, 16, seed=seed_of("half"), lens=[60, 21])
    gw = torch.randn(case["q"].shape, generator=torch.Generator().manual_seed(4))
    feats, sl = case["feats"].to(DEV), case["seqlens"].to(DEV)
    w = case["weight"].to(DEV, torch.float32)
    b = case["bias"].to(DEV, torch.float32)

    def run(dtype):
        leaves = [case[n].to(DEV, torch.float16).to(dtype).requires_grad_(True) for n in ("q", "k", "v")]
        out = flash_spacetime_attention(*leaves, feats, w, b, sl)
        out.backward(gw.to(DEV, torch.float16).to(dtype))
        return out, [x.grad for x in leaves]

    out, grads = run(torch.float16)
    ref_out, ref_grads = run(torch.bfloat16)
    assert out.dtype == torch.float16 and all(g.dtype == torch.float16 for g in grads)
    valid = oracle.valid_row_mask(2, 60, case["seqlens"]).to(DEV)[:, None, :, None]
    assert torch.equal(out, ref_out.to(torch.float16))
    # The bf16 path sees bf16(fp16(x)) operands and a bf16 upstream gradient.
    q64, k64, v64 = (case[n].to(torch.float16).to(torch.bfloat16).double() for n in ("q", "k", "v"))
    ref, _ = oracle.attention_fp64_chunked(q64, k64, v64, case["feats"], w.double().cpu(), b.double().cpu(),
                                           case["seqlens"])
    vm = valid.cpu().expand(ref.shape)
    assert rel_err(out.double().cpu()[vm], ref[vm]) <= 2e-2
    # The float16 result is converted from a temporary bf16 output, which the
    # op does not keep alive for its backward: the rows kernel forms D online,
    # as the bf16 backward does without the forward's output (same N / Z,
    # the schedule's own roundings).
    bq, bk, bv = (case[n].to(DEV, torch.float16).to(torch.bfloat16) for n in ("q", "k", "v"))
    _, ref_lse = flash_spacetime_forward(bq, bk, bv, feats, w, b, sl)
    online = flash_spacetime_backward(bq, bk, bv, feats, w, b, sl, ref_lse,
                                      gw.to(DEV, torch.float16).to(torch.bfloat16))
    for g, r, r_out in zip(grads, online[:3], ref_grads):
        assert torch.equal(g, r.to(torch.float16))
        assert rel_err(g.double().cpu(), r_out.double().cpu()) <= 2e-2


def test_half_launchers_packed_and_qkv():
    gen = torch.Generator().manual_seed(8)
    lens = [40, 7, 19]
    total = sum(lens)
    cu = torch.tensor([0, 40, 47, 66], dtype=torch.int32, device=DEV)
    q, k, v, do = (torch.randn(total, 4, 16, generator=gen).to(DEV, torch.float16) for _ in range(4))
    feats = torch.randn(total, 4, generator=gen).to(DEV)
    w = (torch.randn(16, 32, generator=gen) / 6).to(DEV)
    b = (torch.randn(16, generator=gen) * 0.02).to(DEV)
    out, lse = flash_spacetime_forward(q, k, v, feats, w, b, None, cu_seqlens=cu)
    bq, bk, bv, bdo = (t.to(torch.bfloat16) for t in (q, k, v, do))
    ref_out, ref_lse = flash_spacetime_forward(bq, bk, bv, feats, w, b, None, cu_seqlens=cu)
    assert out.dtype == torch.float16 and torch.equal(out, ref_out.to(torch.float16))
    assert torch.equal(lse, ref_lse)
    grads = flash_spacetime_backward(q, k, v, feats, w, b, None, lse, do, cu_seqlens=cu)
    ref = flash_spacetime_backward(bq, bk, bv, feats, w, b, None, ref_lse, bdo, cu_seqlens=cu)
    for g, r in zip(grads[:3], ref[:3]):
        assert g.dtype == torch.float16 and torch.equal(g, r.to(torch.float16))
    assert torch.equal(grads[3], ref[3]) and torch.equal(grads[4], ref[4])
    assert torch.equal(flash_spacetime_attention_varlen(q, k, v, feats, w, b, cu), out)
    qkv = torch.stack([q, k, v], 1)
    assert torch.equal(flash_spacetime_attention_qkv(qkv, feats, w, b, cu_seqlens=cu), out)
