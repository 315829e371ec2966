"""GPU tests of empty problems through the public operators.

A batch of no events, a batch whose events are all empty, packed events
with no tokens at all, and one-token padded events: forward and backward
run, padding rows (here every row, or none) follow the contract -- outputs
and q/k/v gradients of empty events are exact zeros, and dW / db are zero
when no pair exists. The reference's launchers take the same inputs
(forward.py:222-346, backward.py:488-630).
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from flash_spacetime_amd import flash_spacetime_attention, flash_spacetime_attention_varlen

DEV = "cuda"
DTYPES = [torch.bfloat16, torch.float32]


def _params(dim=32, chans=16):
    gen = torch.Generator().manual_seed(1)
    w = (torch.randn(dim, chans, generator=gen) / 4).to(DEV).requires_grad_(True)
    b = (torch.randn(dim, generator=gen) * 0.02).to(DEV).requires_grad_(True)
    return w, b


def _leaves(shape, dtype, seed=2):
    gen = torch.Generator().manual_seed(seed)
    return [torch.randn(*shape, generator=gen).to(DEV, dtype).requires_grad_(True) for _ in range(3)]


@pytest.mark.parametrize("dtype", DTYPES, ids=["bf16", "fp32"])
@pytest.mark.parametrize("batch,lens", [(0, []), (3, [0, 0, 0])], ids=["no-events", "all-empty"])
def test_padded_empty(dtype, batch, lens):
    length = 24
    q, k, v = _leaves((batch, 4, length, 32), dtype)
    w, b = _params()
    feats = torch.randn(batch, length, 4, device=DEV)
    out = flash_spacetime_attention(q, k, v, feats, w, b, torch.tensor(lens, dtype=torch.int32, device=DEV))
    out.backward(torch.ones_like(out))
    torch.cuda.synchronize()
    assert out.shape == q.shape and (out == 0).all()
    for t in (q, k, v):
        assert t.grad.shape == t.shape and (t.grad == 0).all()
    assert (w.grad == 0).all() and (b.grad == 0).all()


@pytest.mark.parametrize("dtype", DTYPES, ids=["bf16", "fp32"])
def test_packed_no_tokens(dtype):
    q, k, v = _leaves((0, 4, 32), dtype)
    w, b = _params()
    cu = torch.zeros(4, dtype=torch.int32, device=DEV)  # three empty events
    out = flash_spacetime_attention_varlen(q, k, v, torch.zeros(0, 4, device=DEV), w, b, cu)
    out.backward(torch.ones_like(out))
    torch.cuda.synchronize()
    assert out.shape == (0, 4, 32)
    assert all(t.grad.shape == t.shape for t in (q, k, v))
    assert (w.grad == 0).all() and (b.grad == 0).all()


@pytest.mark.parametrize("dtype", DTYPES, ids=["bf16", "fp32"])
def test_padded_single_token_events(dtype):
    """L = 1: each event's only key is the token itself, so out = v + W[:, C/2:] 1
    + b (E of a pair with zero interval is [0..0, 1..1]), dq = dk = 0 and
    dv = dO."""
    q, k, v = _leaves((3, 4, 1, 32), dtype)
    w, b = _params()
    feats = torch.randn(3, 1, 4, device=DEV)
    out = flash_spacetime_attention(q, k, v, feats, w, b, torch.ones(3, dtype=torch.int32, device=DEV))
    want = v.detach().float() + (w.detach()[:, 8:].sum(1) + b.detach())
    tol = 2e-2 if dtype == torch.bfloat16 else 1e-5
    torch.testing.assert_close(out.detach().float(), want, atol=tol, rtol=tol)
    out.backward(torch.ones_like(out))
    torch.cuda.synchronize()
    # One key: the softmax is constant, so q and k get no gradient up to
    # rounding (D = sum p dp / sum p equals dp only to rounding); dv = dO.
    zero_tol = 1e-3 if dtype == torch.bfloat16 else 1e-5
    assert q.grad.float().abs().max() <= zero_tol and k.grad.float().abs().max() <= zero_tol
    torch.testing.assert_close(v.grad.float(), torch.ones(v.shape, device=DEV), atol=tol, rtol=tol)


@pytest.mark.parametrize("dtype", DTYPES, ids=["bf16", "fp32"])
@pytest.mark.parametrize("heads,dim,chans", [(8, 64, 64), (12, 32, 16)], ids=["h8d64c64", "h12d32c16"])
def test_padded_empty_events_beside_others(dtype, heads, dim, chans):
    """Empty events first and last in a padded batch, at the shapes whose
    float32 kernels prefetch rows, positions and u / w~ ahead of a chunk (the
    prefetches of an empty event's single workgroup must not run): the empty
    events' outputs and gradients are exact zeros, and the other event's out,
    dq, dk and dv are bitwise those of the same event run alone."""
    length = 40
    gen = torch.Generator().manual_seed(7)
    q, k, v = (torch.randn(3, heads, length, dim, generator=gen).to(DEV, dtype) for _ in range(3))
    feats = torch.randn(3, length, 4, generator=gen).to(DEV)
    do = torch.randn(3, heads, length, dim, generator=gen).to(DEV, dtype)
    w, b = _params(dim, chans)

    def run(sl, lens):
        leaves = [t[sl].detach().clone().requires_grad_(True) for t in (q, k, v)]
        out = flash_spacetime_attention(*leaves, feats[sl], w, b, torch.tensor(lens, dtype=torch.int32, device=DEV))
        out.backward(do[sl])
        torch.cuda.synchronize()
        return out.detach(), [t.grad for t in leaves]

    out, grads = run(slice(0, 3), [0, 33, 0])
    for e in (0, 2):
        assert (out[e] == 0).all() and all((g[e] == 0).all() for g in grads)
    out1, grads1 = run(slice(1, 2), [33])
    assert torch.equal(out[1:2], out1)
    for g, g1 in zip(grads, grads1):
        assert torch.equal(g[1:2], g1)
