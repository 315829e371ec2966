"""Self-consistency of the bf16 backward: sum_j dS_ij = 0 as the products see it.

The reference keeps rowsum(dS) = 0 per row by forming the softmax row term
D_i = sum_j P dP / sum_j P from the same P and dP that build dS
(backward.py:371-407); README.md:53-73 describes the training failure when
it does not hold. The kernel's `rowsum` output is formed from the same fp32
sums as D and is zero up to one rounding whatever the bf16 dS values were,
so it cannot show this. These tests measure it through dq instead.

Construction: in every event all keys are one vector (k_j = k per head) and
all positions one point (pos_j = pos). Then every logit of a row is the same
number, E_ij = E(0) = [0]*C/2 ++ [1]*C/2 for every pair, and

    dq_i = scale * (sum_j dS_ij k + W sum_j dS_ij E(0) + sigma_i b)
         = scale * sigma_i * (k + W E(0) + b)

where the first two sums are the ones the dQ and H products accumulated
from the bf16 dS values they were fed (plus the kernel's fp32 corrections).
In exact arithmetic sigma_i = 0, so dq_i is pure rounding error, and its
size bounds |sum_j dS_ij| as the products saw it.

Bound. With bf16 round-to-nearest (unit roundoff 2^-8), each dS value fed
to a product is P_j (dP_j - D_c) with D_c the row term at the time (a
P-weighted mean of dP over a subset of the keys, so within [min dP, max dP];
or, when the forward's output is passed, dO . (out - b), the final D up to
the output's rounding) and each correction uses bf16 P_j; the final D lies
in the same range. So

    |sigma_i| <= 2^-8 * (A_i + 4 M_i) + fp32 accumulation
    A_i = sum_j P_j |dP_j - D_i|,   M_i = max_j |dP_j - D_i|

computed here from the float64 oracle's dP (times 1.25 for the kernel's
own bf16 operands, plus n 2^-22 (M_i + |D_i|) for the fp32 sums). The test
asserts |dq_i[d]| <= scale * bound_i * (|k[d]| + |W E(0)|[d] + |b[d]|) * (1 + 2^-7)
(the last factor: dq's own bf16 rounding) on sampled rows of every event.

That worst case grows like the sum of the n rounding errors; the errors
are independent and unbiased (round to nearest even), so their sum is
also held to seven standard deviations of it,

    std_i = 2^-8 sqrt(sum_j P_j^2 ((|dP_j - D_i| + 2 M_i)^2 + (2 M_i)^2) / 3)

(each rounding error uniform within half an ulp <= 2^-8 |x|), which shrinks
like 1 / sqrt(n) and separates rounding noise from a systematic mismatch
between the D that built dS and the one the sums imply.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from flash_spacetime_amd import flash_spacetime_backward, flash_spacetime_forward

DEV = "cuda"


def _constant_key_inputs(batch, length, heads, dim, chans, lens, seed, qk_scale):
    gen = torch.Generator().manual_seed(seed)
    rn = lambda *s: torch.randn(*s, generator=gen)
    q = rn(batch, heads, length, dim) * qk_scale
    k = (rn(batch, heads, 1, dim) * qk_scale).expand(batch, heads, length, dim).contiguous()
    v = rn(batch, heads, length, dim)
    xyz = (torch.rand(batch, 1, 3, generator=gen) - 0.5) * 1000
    t = torch.rand(batch, 1, 1, generator=gen) * 2e4
    feats = torch.cat([xyz, t], -1).expand(batch, length, 4).contiguous()
    w = rn(dim, chans) / chans ** 0.5
    b = rn(dim) * 0.02
    do = rn(batch, heads, length, dim)
    # The kernel's operands are bf16; the bound is computed from the same
    # rounded values.
    q, k, v, do = (x.to(torch.bfloat16) for x in (q, k, v, do))
    return q, k, v, feats, w, b, torch.tensor(lens, dtype=torch.int32), do


def _check(batch, length, heads, dim, chans, lens, seed, qk_scale, rows_per_event, with_out):
    q, k, v, feats, w, b, sl, do = _constant_key_inputs(batch, length, heads, dim, chans, lens, seed, qk_scale)
    g = lambda x: x.to(DEV)
    out, lse = flash_spacetime_forward(g(q), g(k), g(v), g(feats), g(w), g(b), g(sl))
    # with_out: the rows kernel's reference D comes from the forward's output
    # and its sums are corrected once at the end; else D is formed online.
    dq, dk, dv, dw, db = flash_spacetime_backward(g(q), g(k), g(v), g(feats), g(w), g(b), g(sl), lse, g(do),
                                                  out=out if with_out else None)
    torch.cuda.synchronize()
    dq = dq.double().cpu()
    assert torch.isfinite(dq).all()

    scale = dim ** -0.5
    w64, b64 = w.double(), b.double()
    e0 = torch.cat([torch.zeros(chans // 2), torch.ones(chans // 2)]).double()
    r0 = w64 @ e0 + b64  # R(0) = W E(0) + b, the pair feature of every pair
    we0 = (w64 @ e0).abs()
    gen = torch.Generator().manual_seed(seed + 1)
    worst = worst_s = 0.0
    checked = 0
    for bi, n in enumerate(lens):
        rows = torch.randperm(n, generator=gen)[:rows_per_event]
        ve = v[bi, :, :n].double()                      # [H, n, D]
        ge = do[bi, :, rows].double()                   # [H, r, D]
        dp = ge @ ve.transpose(-1, -2) + (ge @ r0)[..., None]  # [H, r, n]; P uniform over the keys
        dmean = dp.mean(-1, keepdim=True)
        dev = (dp - dmean).abs()
        a_i = dev.mean(-1)
        m_i = dev.amax(-1)
        slack = n * 2.0 ** -22 * (m_i + dmean[..., 0].abs())
        bound = 1.25 * 2.0 ** -8 * (a_i + 4 * m_i) + slack  # [H, r]
        p2 = 1.0 / n ** 2
        std = 2.0 ** -8 * torch.sqrt(p2 * (((dev + 2 * m_i[..., None]) ** 2).sum(-1) + n * (2 * m_i) ** 2) / 3)
        stat = 1.25 * 7.0 * std + slack
        kvec = k[bi, :, 0].double().abs()               # [H, D]
        weight = (kvec[:, None, :] + we0 + b64.abs()) * (1 + 2.0 ** -7) * scale
        got = dq[bi, :, rows].abs()
        ratio = (got / (bound[..., None] * weight)).max().item()
        ratio_s = (got / (stat[..., None] * weight)).max().item()
        worst = max(worst, ratio)
        worst_s = max(worst_s, ratio_s)
        checked += got.numel()
        assert ratio <= 1.0, f"event {bi} (n={n}): |dq| exceeds the worst-case rounding bound (ratio {ratio:.3f})"
        assert ratio_s <= 1.0, f"event {bi} (n={n}): |dq| exceeds 7 std of the rounding (ratio {ratio_s:.3f})"
    print(f"constant-key self-consistency: {checked} dq entries, worst |dq| / worst-case bound = {worst:.3e}, "
          f"/ 7-std bound = {worst_s:.3e}")


WITH_OUT = pytest.mark.parametrize("with_out", [False, True], ids=["online_d", "reference_d"])


@WITH_OUT
def test_rowsum_via_dq_cfg2_shape(with_out):
    gen = torch.Generator().manual_seed(5)
    lens = torch.randint(16, 769, (256,), generator=gen).tolist()
    lens[0], lens[1] = 768, 16
    _check(256, 768, 12, 32, 16, lens, 50, 1.0, rows_per_event=8, with_out=with_out)


@WITH_OUT
def test_rowsum_via_dq_cfg4_x30(with_out):
    _check(8, 4096, 8, 64, 64, [4096] * 8, 60, 30.0, rows_per_event=48, with_out=with_out)
