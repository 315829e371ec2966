"""GPU tests of the packed (varlen, uncapped) path.

Re-expresses the reference's test_varlen.py: packed == padded on the same
events, packed fwd+bwd against the float64 oracle, bitwise determinism, and
the uncapped-length smoke with its memory ceiling; adds a BASELINE config-3
style batch (lognormal lengths, >= 1% single-token events).
"""

import math

import pytest
import torch

import oracle
from tests._cases import FLAGS, make_packed, rel_err, seed_of

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from flash_spacetime_amd import flash_spacetime_attention, flash_spacetime_attention_varlen

LENGTH_MIXES = [[7], [1, 1, 1], [17, 64, 3], [200, 33, 1, 128], [331, 800, 65]]


def _pad(x: torch.Tensor, lengths, feats: bool = False) -> torch.Tensor:
    """Packed [T, ...] -> padded [B, H, L, D] (or [B, L, F] for feats)."""
    length = max(lengths)
    chunks = torch.split(x, list(lengths))
    if feats:
        out = x.new_zeros(len(lengths), length, x.shape[-1])
        for i, c in enumerate(chunks):
            out[i, : c.shape[0]] = c
        return out
    out = x.new_zeros(len(lengths), length, x.shape[1], x.shape[2])
    for i, c in enumerate(chunks):
        out[i, : c.shape[0]] = c
    return out.permute(0, 2, 1, 3).contiguous()


def _unpad(padded: torch.Tensor, lengths) -> torch.Tensor:
    return torch.cat([padded[i, :, :n].permute(1, 0, 2) for i, n in enumerate(lengths)], 0)


@pytest.mark.parametrize("lengths", LENGTH_MIXES, ids=lambda l: "-".join(map(str, l)))
@pytest.mark.parametrize("flags", FLAGS, ids=lambda f: f"attn{int(f[0])}act{int(f[1])}")
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_varlen_matches_padded(lengths, flags, dtype):
    """Packed and padded paths agree on identical events (test_varlen.py:103-146)."""
    case = make_packed(lengths, 4, 48, 48, seed_of("vp", tuple(lengths), flags))
    dev = "cuda"
    seqlens = torch.tensor(lengths, device=dev)
    out_v = flash_spacetime_attention_varlen(
        case["q"].to(dev, dtype), case["k"].to(dev, dtype), case["v"].to(dev, dtype),
        case["feats"].to(dev), case["weight"].to(dev, dtype), case["bias"].to(dev, dtype),
        case["cu"].to(dev), use_attn_bias=flags[0], use_activation_bias=flags[1],
    )
    out_p = flash_spacetime_attention(
        _pad(case["q"], lengths).to(dev, dtype), _pad(case["k"], lengths).to(dev, dtype),
        _pad(case["v"], lengths).to(dev, dtype), _pad(case["feats"], lengths, True).to(dev),
        case["weight"].to(dev, dtype), case["bias"].to(dev, dtype), seqlens,
        use_attn_bias=flags[0], use_activation_bias=flags[1],
    )
    atol, rtol = (2e-2, 1e-2) if dtype is torch.bfloat16 else (1e-5, 1e-4)
    torch.testing.assert_close(out_v, _unpad(out_p, lengths), atol=atol, rtol=rtol)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_many_events_packed_matches_padded(dtype):
    """5000 short events, fwd+bwd: the packed work list's event lookup takes
    three rounds of the wave-wide search (more than 64 x 64 events), the
    padded bf16 rows kernel's two; both layouts agree on every event."""
    gen = torch.Generator().manual_seed(5000)
    lengths = torch.randint(1, 25, (5000,), generator=gen).tolist()
    case = make_packed(lengths, 2, 16, 16, seed_of("many", dtype))
    dev = "cuda"
    packed = {k: case[k].to(dev, dtype).requires_grad_(True) for k in ("q", "k", "v")}
    padded = {k: _pad(case[k], lengths).to(dev, dtype).requires_grad_(True) for k in ("q", "k", "v")}
    w, b = case["weight"].to(dev, dtype), case["bias"].to(dev, dtype)
    out_v = flash_spacetime_attention_varlen(packed["q"], packed["k"], packed["v"], case["feats"].to(dev), w, b,
                                             case["cu"].to(dev))
    out_p = flash_spacetime_attention(padded["q"], padded["k"], padded["v"], _pad(case["feats"], lengths, True).to(dev),
                                      w, b, torch.tensor(lengths, device=dev))
    gen_do = torch.Generator().manual_seed(5001)
    do = torch.randn(out_v.shape, generator=gen_do, dtype=torch.float64)
    out_v.backward(do.to(dev, dtype))
    out_p.backward(_pad(do, lengths).to(dev, dtype))
    atol, rtol = (2e-2, 1e-2) if dtype is torch.bfloat16 else (1e-5, 1e-4)
    torch.testing.assert_close(out_v, _unpad(out_p, lengths), atol=atol, rtol=rtol)
    bound = 1e-2 if dtype is torch.bfloat16 else 1e-5
    for key in ("q", "k", "v"):
        err = rel_err(packed[key].grad, _unpad(padded[key].grad, lengths))
        assert err <= bound, f"grad {key}: relative error {err:.2e}"


@pytest.mark.parametrize("lengths", LENGTH_MIXES[2:], ids=lambda l: "-".join(map(str, l)))
@pytest.mark.parametrize("flags", FLAGS[:2], ids=["attn1act1", "attn1act0"])
def test_varlen_matches_oracle(lengths, flags):
    """Packed fwd+bwd against the float64 oracle (test_varlen.py:149-225)."""
    case = make_packed(lengths, 4, 48, 48, seed_of("vo", tuple(lengths), flags))
    dev = "cuda"
    leaves = {k: case[k].to(dev, torch.float32).requires_grad_(True) for k in ("q", "k", "v")}
    leaves["W"] = case["weight"].to(dev, torch.float32).requires_grad_(True)
    leaves["b"] = case["bias"].to(dev, torch.float32).requires_grad_(True)
    out = flash_spacetime_attention_varlen(
        leaves["q"], leaves["k"], leaves["v"], case["feats"].to(dev), leaves["W"], leaves["b"],
        case["cu"].to(dev), use_attn_bias=flags[0], use_activation_bias=flags[1],
    )
    (out.double().pow(2).sum() * 0.5).backward()
    ref, _ = oracle.attention_fp64_chunked(
        case["q"], case["k"], case["v"], case["feats"], case["weight"], case["bias"],
        cu_seqlens=case["cu"], use_attn_bias=flags[0], use_activation_bias=flags[1],
    )
    torch.testing.assert_close(out.detach().double().cpu(), ref, atol=5e-3, rtol=1e-3)
    dq, dk, dv, dW, db = oracle.backward_fp64_chunked(
        case["q"], case["k"], case["v"], case["feats"], case["weight"], case["bias"], ref,
        cu_seqlens=case["cu"], use_attn_bias=flags[0], use_activation_bias=flags[1],
    )
    for key, want in (("q", dq), ("k", dk), ("v", dv), ("W", dW), ("b", db)):
        got = leaves[key].grad
        assert got is not None
        torch.testing.assert_close(got.double().cpu(), want, atol=5e-2, rtol=5e-3,
                                   msg=lambda m, key=key: f"grad {key}: {m}")


def test_varlen_deterministic():
    """Two identical packed fwd+bwd runs are bitwise identical (test_varlen.py:228-248)."""
    case = make_packed([64, 17, 200], 16, 48, 48, 99)
    dev = "cuda"
    results = []
    for _ in range(2):
        q = case["q"].to(dev, torch.float32).requires_grad_(True)
        w = case["weight"].to(dev, torch.float32).requires_grad_(True)
        out = flash_spacetime_attention_varlen(
            q, case["k"].to(dev, torch.float32), case["v"].to(dev, torch.float32),
            case["feats"].to(dev), w, case["bias"].to(dev, torch.float32), case["cu"].to(dev),
        )
        out.sum().backward()
        results.append((out.detach().clone(), q.grad.clone(), w.grad.clone()))
    for a, b in zip(results[0], results[1]):
        assert torch.equal(a, b)


def test_uncapped_lengths_smoke():
    """A 6000-token event in < 0.5 GiB of transient memory (test_varlen.py:251-282)."""
    lengths = [6000, 137, 1503]
    case = make_packed(lengths, 16, 48, 48, 7)
    dev = "cuda"
    q = case["q"].to(dev, torch.bfloat16).requires_grad_(True)
    w = case["weight"].to(dev, torch.bfloat16).requires_grad_(True)
    k = case["k"].to(dev, torch.bfloat16)
    v = case["v"].to(dev, torch.bfloat16)
    feats = case["feats"].to(dev)
    b = case["bias"].to(dev, torch.bfloat16)
    cu = case["cu"].to(dev)
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    out = flash_spacetime_attention_varlen(q, k, v, feats, w, b, cu)
    out.sum().backward()
    torch.cuda.synchronize()
    peak = (torch.cuda.max_memory_allocated() - base) / 2 ** 30
    assert torch.isfinite(out).all()
    assert q.grad is not None and torch.isfinite(q.grad).all()
    assert w.grad is not None and torch.isfinite(w.grad).all()
    assert peak < 0.5, f"packed fwd+bwd peak {peak:.2f} GiB"


def _lognormal_lengths(n_events: int, seed: int, cap: int = 3000):
    gen = torch.Generator().manual_seed(seed)
    lens = torch.exp(5.0 + torch.randn(n_events, generator=gen, dtype=torch.float64)).round()
    lens = lens.clamp(1, cap).long()
    ones = torch.randperm(n_events, generator=gen)[: max(1, math.ceil(0.01 * n_events))]
    lens[ones] = 1
    return lens.tolist()


def test_config3_style_batch_against_oracle():
    """BASELINE cfg3 distribution (lognormal lengths, >= 1% single-token events),
    H=12, D=32, C=16, bf16, at 48 events: fwd+bwd within 2e-2 of float64."""
    lengths = _lognormal_lengths(48, 3, cap=600)
    case = make_packed(lengths, 12, 32, 16, seed_of("cfg3", 48))
    dev = "cuda"
    leaves = {k: case[k].to(dev, torch.bfloat16).requires_grad_(True) for k in ("q", "k", "v")}
    w = case["weight"].to(dev, torch.float32).requires_grad_(True)
    b = case["bias"].to(dev, torch.float32).requires_grad_(True)
    out = flash_spacetime_attention_varlen(leaves["q"], leaves["k"], leaves["v"], case["feats"].to(dev),
                                           w, b, case["cu"].to(dev))
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(4), dtype=torch.float64)
    out.backward(g.to(dev, out.dtype))
    ref, _ = oracle.attention_fp64_chunked(case["q"], case["k"], case["v"], case["feats"], case["weight"],
                                           case["bias"], cu_seqlens=case["cu"])
    assert rel_err(out.detach().cpu(), ref) <= 2e-2
    grads = oracle.backward_fp64_chunked(case["q"], case["k"], case["v"], case["feats"], case["weight"],
                                         case["bias"], g.to(torch.bfloat16).double(),
                                         cu_seqlens=case["cu"])
    for name, got, want in zip("q k v W b".split(), (leaves["q"].grad, leaves["k"].grad, leaves["v"].grad,
                                                     w.grad, b.grad), grads):
        assert rel_err(got.cpu(), want) <= 2e-2, name


def test_empty_and_single_token_events():
    """Zero-length events in the packed list are skipped; length-1 events give
    out = v + W[:, C/2:] 1 + b (E of a token with itself is [0..0, 1..1])."""
    lengths = [1, 0, 5, 0, 1]
    case = make_packed(lengths, 4, 32, 16, 5)
    dev = "cuda"
    out = flash_spacetime_attention_varlen(
        case["q"].to(dev, torch.float32), case["k"].to(dev, torch.float32), case["v"].to(dev, torch.float32),
        case["feats"].to(dev), case["weight"].to(dev, torch.float32), case["bias"].to(dev, torch.float32),
        case["cu"].to(dev),
    ).cpu().double()
    want = case["v"] + case["weight"][:, 8:].sum(1) + case["bias"]
    torch.testing.assert_close(out[0], want[0], atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(out[-1], want[-1], atol=1e-5, rtol=1e-5)
