"""GPU checks at the BASELINE configurations' full sizes.

The float64 oracle cannot evaluate these shapes in test time, so the full
runs are checked through properties that do not depend on size, and events
that are small enough are compared with the oracle one by one (events are
independent, so an event's rows must equal the oracle on that event alone):

* cfg2 (B=256, L=768, H=12, D=32, C=16, bf16, lengths U{16..768}) and cfg3
  (4096 packed events, lognormal lengths in [1, 3000], >= 1 % of length 1):
  finite results, padding rows exactly zero, sum_j dS_ij = 0 per row within
  fp32 rounding, bitwise determinism, and sampled events against the oracle;
* cfg4 (B=8, L=4096, H=8, D=C=64, q and k x30, fp32 and bf16): finite
  results and gradients, the row sum of dS, and the padded result equal to
  the packed one on the same events.
"""

import math

import pytest
import torch

import oracle
from tests._cases import rel_err

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from flash_spacetime_amd import (
        flash_spacetime_attention_varlen, flash_spacetime_backward, flash_spacetime_forward,
    )

DEV = "cuda"


def _inputs_padded(batch, length, heads, dim, chans, lens, seed, dtype, qk_scale=1.0):
    gen = torch.Generator().manual_seed(seed)
    rn = lambda *s: torch.randn(*s, generator=gen)
    q = (rn(batch, heads, length, dim) * qk_scale).to(DEV, dtype)
    k = (rn(batch, heads, length, dim) * qk_scale).to(DEV, dtype)
    v = rn(batch, heads, length, dim).to(DEV, dtype)
    xyz = (torch.rand(batch, length, 3, generator=gen) - 0.5) * 1000
    t = torch.rand(batch, length, 1, generator=gen) * 2e4
    feats = torch.cat([xyz, t], -1).to(DEV)
    w = (rn(dim, chans) / chans ** 0.5).to(DEV)
    b = (rn(dim) * 0.02).to(DEV)
    do = rn(batch, heads, length, dim).to(DEV, dtype)
    return q, k, v, feats, w, b, torch.tensor(lens, dtype=torch.int32, device=DEV), do


def _fwd_bwd(q, k, v, feats, w, b, seqlens=None, cu=None, do=None):
    out, lse = flash_spacetime_forward(q, k, v, feats, w, b, seqlens, cu_seqlens=cu)
    rowsum = torch.full(lse.shape, float("nan"), device=DEV)
    grads = flash_spacetime_backward(q, k, v, feats, w, b, seqlens, lse, do, cu_seqlens=cu, rowsum=rowsum)
    torch.cuda.synchronize()
    return out, lse, grads, rowsum


def _rowsum_bound(n, do, v):
    # n fp32 terms of |P (dP - D)| <= |dO| (|v| + |W E| + |b|) each.
    return 64 * 2.0 ** -23 * n * do.float().abs().max().item() * (v.float().abs().max().item() + 10.0)


def _check_event_against_oracle(q, k, v, feats, w, b, out, grads, do, sl, packed_tok0=None):
    """One event, sliced from the batch, against the float64 oracle."""
    if packed_tok0 is None:
        bi, n = sl
        ev = lambda x: x[bi:bi + 1, :, :n].double().cpu()
        fe = feats[bi:bi + 1, :n].double().cpu()
        o, dq, dk, dv = ev(out), ev(grads[0]), ev(grads[1]), ev(grads[2])
        g = ev(do)
        qe, ke, ve = ev(q), ev(k), ev(v)
    else:
        t0, n = packed_tok0, sl
        ev = lambda x: x[t0:t0 + n].double().cpu().permute(1, 0, 2).unsqueeze(0)
        fe = feats[t0:t0 + n].double().cpu().unsqueeze(0)
        o, dq, dk, dv = ev(out), ev(grads[0]), ev(grads[1]), ev(grads[2])
        g = ev(do)
        qe, ke, ve = ev(q), ev(k), ev(v)
    leaves = [x.clone().requires_grad_(True) for x in (qe, ke, ve)]
    ref = oracle.attention(*leaves, fe, w.double().cpu(), b.double().cpu())
    ref.backward(g)
    assert rel_err(o, ref.detach()) <= 2e-2
    for got, leaf in zip((dq, dk, dv), leaves):
        assert rel_err(got, leaf.grad) <= 2e-2


def test_cfg2_full_size():
    gen = torch.Generator().manual_seed(2)
    lens = torch.randint(16, 769, (256,), generator=gen).tolist()
    lens[0], lens[1] = 16, 768
    q, k, v, feats, w, b, sl, do = _inputs_padded(256, 768, 12, 32, 16, lens, 22, torch.bfloat16)
    out, lse, grads, rowsum = _fwd_bwd(q, k, v, feats, w, b, sl, do=do)
    valid = (torch.arange(768, device=DEV)[None, :] < sl[:, None].long())
    vm = valid[:, None, :, None].expand(out.shape)
    assert torch.isfinite(out).all() and (out[~vm] == 0).all()
    for gr in grads[:3]:
        assert torch.isfinite(gr).all() and (gr[~vm] == 0).all()
    rs = rowsum[valid[:, None, :].expand(rowsum.shape)]
    assert rs.abs().max().item() <= _rowsum_bound(768, do, v)
    again = _fwd_bwd(q, k, v, feats, w, b, sl, do=do)
    assert torch.equal(out, again[0]) and all(torch.equal(a, c) for a, c in zip(grads[:4], again[2][:4]))
    _check_event_against_oracle(q, k, v, feats, w, b, out, grads, do, (0, lens[0]))
    _check_event_against_oracle(q, k, v, feats, w, b, out, grads, do, (2, lens[2]))


def _lognormal_lengths(n_events, seed, cap=3000):
    gen = torch.Generator().manual_seed(seed)
    lens = torch.exp(5.0 + torch.randn(n_events, generator=gen, dtype=torch.float64)).round().clamp(1, cap).long()
    ones = torch.randperm(n_events, generator=gen)[: max(1, math.ceil(0.01 * n_events))]
    lens[ones] = 1
    return lens.tolist()


def test_cfg3_full_size():
    lens = _lognormal_lengths(4096, 3)
    total = sum(lens)
    gen = torch.Generator().manual_seed(33)
    rn = lambda *s: torch.randn(*s, generator=gen)
    q, k, v, do = (rn(total, 12, 32).to(DEV, torch.bfloat16) for _ in range(4))
    xyz = (torch.rand(total, 3, generator=gen) - 0.5) * 1000
    t = torch.rand(total, 1, generator=gen) * 2e4
    feats = torch.cat([xyz, t], -1).to(DEV)
    w = (rn(32, 16) / 4).to(DEV)
    b = (rn(32) * 0.02).to(DEV)
    cu_list = [0]
    for n in lens:
        cu_list.append(cu_list[-1] + n)
    cu = torch.tensor(cu_list, dtype=torch.int32, device=DEV)
    out, lse, grads, rowsum = _fwd_bwd(q, k, v, feats, w, b, cu=cu, do=do)
    assert torch.isfinite(out).all() and all(torch.isfinite(gr).all() for gr in grads[:4])
    assert rowsum.abs().max().item() <= _rowsum_bound(max(lens), do, v)
    again = _fwd_bwd(q, k, v, feats, w, b, cu=cu, do=do)
    assert torch.equal(out, again[0]) and all(torch.equal(a, c) for a, c in zip(grads[:4], again[2][:4]))
    # Single-token events: out = v + W[:, C/2:] 1 + b (E of a token with itself).
    one = lens.index(1)
    want = v[cu_list[one]].float() + (w[:, 8:].sum(1) + b)[None, :]
    torch.testing.assert_close(out[cu_list[one]].float(), want, atol=3e-2, rtol=2e-2)
    # Two events of moderate length against the oracle.
    picks = [i for i, n in enumerate(lens) if 50 <= n <= 200][:2]
    for i in picks:
        _check_event_against_oracle(q, k, v, feats, w, b, out, grads, do, lens[i], packed_tok0=cu_list[i])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_cfg4_full_size(dtype):
    lens = [4096] * 8
    q, k, v, feats, w, b, sl, do = _inputs_padded(8, 4096, 8, 64, 64, lens, 44, dtype, qk_scale=30.0)
    out, lse, grads, rowsum = _fwd_bwd(q, k, v, feats, w, b, sl, do=do)
    assert torch.isfinite(out).all() and torch.isfinite(lse).all()
    for gr in grads[:4]:
        assert torch.isfinite(gr).all()
    assert rowsum.abs().max().item() <= _rowsum_bound(4096, do, v)
    # The same events packed: rows agree with the padded run.
    pk = lambda x: x.transpose(1, 2).reshape(-1, x.shape[1], x.shape[3]).contiguous()
    cu = torch.arange(0, 8 * 4096 + 1, 4096, dtype=torch.int32, device=DEV)
    out_p, _, grads_p, _ = _fwd_bwd(pk(q), pk(k), pk(v), feats.reshape(-1, 4), w, b, cu=cu, do=pk(do))
    atol, rtol = (2e-2, 1e-2) if dtype == torch.bfloat16 else (1e-5, 1e-4)
    torch.testing.assert_close(out_p, pk(out), atol=atol, rtol=rtol)
    for a, c in zip(grads_p[:3], grads[:3]):
        assert rel_err(a, pk(c)) <= (1e-2 if dtype == torch.bfloat16 else 1e-4)
