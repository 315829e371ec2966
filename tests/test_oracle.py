"""CPU tests that pin the oracle before it is trusted as the parity checker.

Each oracle function is checked against something it was not derived from:
golden vectors written by the reference's own spec module
(tests/golden/make_golden.py), closed forms, a scalar brute force in plain
Python, and autograd / gradcheck for the closed-form backward. The last
tests plant a plausible mistake in the oracle and assert the checks notice.
"""

import math
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from oracle import spec

GOLDEN = np.load(Path(__file__).parent / "golden" / "reference_spec_vectors.npz")
FLAGS = [(True, True), (True, False), (False, True), (False, False)]


def _t(name, dtype=torch.float64):
    return torch.from_numpy(GOLDEN[name]).to(dtype)


# ----------------------------------------------------------------- constants


def test_time_scale_is_18():
    assert oracle.TIME_SCALE == 18.0
    assert float(np.float32(oracle.TIME_SCALE)) == 18.0
    assert GOLDEN["time_scale"][0] == oracle.TIME_SCALE


@pytest.mark.parametrize("c", [16, 32, 48, 64])
def test_frequency_ladder_matches_reference(c):
    """Bitwise equal to the reference's ladder except where the reference's
    fp32 exp was not correctly rounded; there it is the correctly rounded
    value, one ulp away."""
    got = oracle.frequencies(c).numpy()
    want = GOLDEN[f"freqs_C{c}"]
    assert got.dtype == np.float32
    ulps = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
    assert ulps.max() <= 1
    # Wherever they differ, the oracle holds the correctly rounded exp of the
    # same fp32 argument (the argument itself is reproduced bitwise).
    half = np.float32(c / 2)
    arg = np.arange(c // 2, dtype=np.float32) * (-(np.float32(math.log(1e4)) / half))
    exact = np.array([math.exp(float(a)) for a in arg])
    for i in np.nonzero(ulps)[0]:
        assert abs(float(got[i]) - exact[i]) < abs(float(want[i]) - exact[i])
    if c < 64:
        np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("c", [16, 32, 48, 64])
def test_frequency_ladder_closed_form(c):
    got = oracle.frequencies(c).double().numpy()
    exact = np.array([10000.0 ** (-i / (c / 2)) for i in range(c // 2)])
    # fp32 evaluation: the rounded fp32 step is multiplied by i, so the
    # exponent (hence the relative error) may be off by about i ulps.
    bound = (np.arange(c // 2) + 2) * 2.0 ** -23
    assert np.all(np.abs(got / exact - 1) < bound)
    assert got[0] == 1.0


# ------------------------------------------------------------ pair geometry


def _scalar_embedding(pi, pj, c):
    """E_ij of one pair in binary64 with plain-Python math (brute force)."""
    dx, dy, dz = pi[0] - pj[0], pi[1] - pj[1], pi[2] - pj[2]
    dt = (pi[3] - pj[3]) * 18.0
    interval = dx * dx + dy * dy + dz * dz - dt * dt
    sd = math.copysign(math.sqrt(abs(interval)), interval) if interval != 0 else 0.0
    x = 1024.0 * min(max(sd, -4.0), 4.0)
    freqs = [float(f) for f in oracle.frequencies(c).tolist()]
    return [math.sin(x * f) for f in freqs] + [math.cos(x * f) for f in freqs]


def test_embedding_diagonal_is_zero_angle():
    feats = torch.randn(2, 9, 5, dtype=torch.float64)
    emb = oracle.pair_embedding(feats, 16)
    diag = emb[:, torch.arange(9), torch.arange(9)]
    expect = torch.cat([torch.zeros(8), torch.ones(8)]).double()
    assert torch.equal(diag, expect.expand_as(diag))


def test_angle_saturates_exactly_and_is_symmetric():
    gen = torch.Generator().manual_seed(3)
    xyz = (torch.rand(1, 64, 3, generator=gen, dtype=torch.float64) - 0.5) * 1000
    t = torch.rand(1, 64, 1, generator=gen, dtype=torch.float64) * 2e4
    feats = torch.cat([xyz, t], -1)
    x = oracle.pair_angle(feats)
    off = ~torch.eye(64, dtype=torch.bool)
    assert torch.equal(x, x.transpose(1, 2))
    # raw detector units: every off-diagonal pair is far outside the clip
    assert torch.all(x[0][off].abs() == 4096.0)
    # fp32 feats give the same exact saturated angle
    x32 = oracle.pair_angle(feats.float())
    assert torch.all(x32[0][off].abs() == 4096.0)


def test_light_like_pair_has_zero_angle():
    feats = torch.zeros(1, 2, 4, dtype=torch.float64)
    feats[0, 1] = torch.tensor([18.0, 0.0, 0.0, 1.0])
    x = oracle.pair_angle(feats)
    assert x[0, 0, 1] == 0.0 and x[0, 1, 0] == 0.0
    spacelike = feats.clone()
    spacelike[0, 1, 0] = 18.5
    timelike = feats.clone()
    timelike[0, 1, 0] = 17.5
    assert oracle.pair_angle(spacelike)[0, 0, 1] > 0
    assert oracle.pair_angle(timelike)[0, 0, 1] < 0


def test_embedding_bruteforce_scalar():
    gen = torch.Generator().manual_seed(11)
    feats = torch.randn(1, 12, 4, generator=gen, dtype=torch.float64) * 0.3
    for c in (16, 48):
        emb = oracle.pair_embedding(feats, c)
        f = feats[0].tolist()
        for i in range(12):
            for j in range(12):
                ref = _scalar_embedding(f[i], f[j], c)
                np.testing.assert_allclose(emb[0, i, j].numpy(), ref, rtol=0, atol=1e-12)


@pytest.mark.parametrize("case", ["n16", "r16", "n32"])
@pytest.mark.parametrize("tag", ["f64", "f32", "bf16"])
def test_pair_features_match_reference_vectors(case, tag):
    dt = {"f64": torch.float64, "f32": torch.float32, "bf16": torch.bfloat16}[tag]
    fdt = torch.float64 if dt == torch.float64 else torch.float32
    rel = oracle.pair_features(
        _t(f"{case}_feats", fdt), _t(f"{case}_weight", dt), _t(f"{case}_bias", dt)
    )
    want = GOLDEN[f"{case}_rel_{tag}"]
    np.testing.assert_array_equal(rel.float().numpy() if dt == torch.bfloat16 else rel.numpy(), want)


@pytest.mark.parametrize("case", ["n16", "r16", "n32"])
def test_pair_mask_matches_reference_vectors(case):
    seqlens = torch.from_numpy(GOLDEN[f"{case}_seqlens"])
    b, l = GOLDEN[f"{case}_feats"].shape[:2]
    mask = oracle.float_padding_mask(oracle.valid_row_mask(b, l, seqlens), torch.float32)
    np.testing.assert_array_equal(oracle.pair_mask(mask).numpy(), GOLDEN[f"{case}_pairmask"])


# ------------------------------------------------------------------ forward


@pytest.mark.parametrize("case", ["n16", "r16", "n32"])
@pytest.mark.parametrize("tag", ["f64", "f32", "bf16"])
@pytest.mark.parametrize("flags", FLAGS)
def test_attention_matches_reference_vectors(case, tag, flags):
    dt = {"f64": torch.float64, "f32": torch.float32, "bf16": torch.bfloat16}[tag]
    fdt = torch.float64 if dt == torch.float64 else torch.float32
    seqlens = torch.from_numpy(GOLDEN[f"{case}_seqlens"])
    b, l = GOLDEN[f"{case}_feats"].shape[:2]
    mask = oracle.float_padding_mask(oracle.valid_row_mask(b, l, seqlens), torch.float32)
    out = oracle.attention(
        _t(f"{case}_q", dt), _t(f"{case}_k", dt), _t(f"{case}_v", dt),
        _t(f"{case}_feats", fdt), _t(f"{case}_weight", dt), _t(f"{case}_bias", dt),
        key_padding_mask=mask, use_attn_bias=flags[0], use_activation_bias=flags[1],
    )
    want = GOLDEN[f"{case}_out_{tag}_{int(flags[0])}{int(flags[1])}"]
    got = out.float().numpy() if dt == torch.bfloat16 else out.numpy()
    np.testing.assert_array_equal(got, want)


def _bruteforce_attention(q, k, v, feats, weight, bias, scale, flags):
    """Scalar triple loops over (head, row, key) in plain Python floats."""
    bsz, heads, length, dim = len(q), len(q[0]), len(q[0][0]), len(q[0][0][0])
    c = len(weight[0])
    out = np.zeros((bsz, heads, length, dim))
    for b in range(bsz):
        f = feats[b].tolist()
        emb = [[_scalar_embedding(f[i], f[j], c) for j in range(length)] for i in range(length)]
        rel = [[[sum(weight[d][cc] * emb[i][j][cc] for cc in range(c)) + bias[d]
                 for d in range(dim)] for j in range(length)] for i in range(length)]
        for h in range(heads):
            for i in range(length):
                qt = [scale * q[b][h][i][d] for d in range(dim)]
                logits = []
                for j in range(length):
                    s = sum(qt[d] * k[b][h][j][d] for d in range(dim))
                    if flags[0]:
                        s += sum(qt[d] * rel[i][j][d] for d in range(dim))
                    logits.append(s)
                m = max(logits)
                w = [math.exp(s - m) for s in logits]
                z = sum(w)
                for d in range(dim):
                    acc = sum(w[j] / z * v[b][h][j][d] for j in range(length))
                    if flags[1]:
                        acc += sum(w[j] / z * rel[i][j][d] for j in range(length))
                    out[b, h, i, d] = acc
    return out


@pytest.mark.parametrize("flags", FLAGS)
def test_attention_bruteforce_c_ne_d(flags):
    gen = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn(1, 2, 5, 4, generator=gen, dtype=torch.float64) for _ in range(3))
    feats = torch.randn(1, 5, 4, generator=gen, dtype=torch.float64) * 0.2
    weight = torch.randn(4, 6, generator=gen, dtype=torch.float64)
    bias = torch.randn(4, generator=gen, dtype=torch.float64)
    got = oracle.attention(q, k, v, feats, weight, bias, scale=0.7,
                           use_attn_bias=flags[0], use_activation_bias=flags[1])
    want = _bruteforce_attention(q.tolist(), k.tolist(), v.tolist(), feats, weight.tolist(),
                                 bias.tolist(), 0.7, flags)
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-12, atol=1e-12)


def test_flags_off_is_plain_attention():
    gen = torch.Generator().manual_seed(6)
    q, k, v = (torch.randn(2, 3, 11, 16, generator=gen, dtype=torch.float64) for _ in range(3))
    feats = torch.randn(2, 11, 5, generator=gen, dtype=torch.float64)
    w = torch.randn(16, 8, generator=gen, dtype=torch.float64)
    got = oracle.attention(q, k, v, feats, w, None, use_attn_bias=False, use_activation_bias=False)
    want = torch.nn.functional.scaled_dot_product_attention(q, k, v)
    torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-12)
    zero = oracle.attention(q, k, v, feats, torch.zeros_like(w), torch.zeros(16, dtype=torch.float64))
    torch.testing.assert_close(zero, want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("c", [16, 48])
def test_single_token_event_closed_form(c):
    gen = torch.Generator().manual_seed(c)
    d = 32
    q, k, v = (torch.randn(3, 2, 1, d, generator=gen, dtype=torch.float64) for _ in range(3))
    feats = torch.randn(3, 1, 4, generator=gen, dtype=torch.float64)
    w = torch.randn(d, c, generator=gen, dtype=torch.float64)
    b = torch.randn(d, generator=gen, dtype=torch.float64)
    out = oracle.attention(q, k, v, feats, w, b)
    want = v + w[:, c // 2:].sum(1) + b
    torch.testing.assert_close(out, want, rtol=1e-12, atol=1e-12)


def test_bias_shift_invariance_with_logit_term_only():
    gen = torch.Generator().manual_seed(8)
    q, k, v = (torch.randn(2, 2, 9, 16, generator=gen, dtype=torch.float64) for _ in range(3))
    feats = torch.randn(2, 9, 4, generator=gen, dtype=torch.float64)
    w = torch.randn(16, 16, generator=gen, dtype=torch.float64)
    b1, b2 = (torch.randn(16, generator=gen, dtype=torch.float64) for _ in range(2))
    o1 = oracle.attention(q, k, v, feats, w, b1, use_activation_bias=False)
    o2 = oracle.attention(q, k, v, feats, w, b2 * 5, use_activation_bias=False)
    torch.testing.assert_close(o1, o2, rtol=1e-10, atol=1e-10)


# -------------------------------------------------- chunked fp64 evaluators


def _padded_case(bsz, length, heads, d, c, seed, lens=None):
    gen = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(bsz, heads, length, d, generator=gen, dtype=torch.float64) for _ in range(3))
    feats = torch.randn(bsz, length, 5, generator=gen, dtype=torch.float64)
    w = torch.randn(d, c, generator=gen, dtype=torch.float64) / c ** 0.5
    b = torch.randn(d, generator=gen, dtype=torch.float64)
    seqlens = torch.tensor(lens if lens is not None else [length] * bsz)
    return q, k, v, feats, w, b, seqlens


@pytest.mark.parametrize("flags", FLAGS)
def test_chunked_forward_matches_eager(flags):
    q, k, v, feats, w, b, seqlens = _padded_case(3, 23, 2, 16, 8, 21, lens=[23, 7, 1])
    valid = oracle.valid_row_mask(3, 23, seqlens)
    mask = oracle.float_padding_mask(valid, torch.float64)
    eager = oracle.attention(q, k, v, feats, w, b, key_padding_mask=mask,
                             use_attn_bias=flags[0], use_activation_bias=flags[1])
    out, lse = oracle.attention_fp64_chunked(q, k, v, feats, w, b, seqlens,
                                             use_attn_bias=flags[0], use_activation_bias=flags[1],
                                             row_block=5)
    vm = valid[:, None, :, None].expand_as(out)
    torch.testing.assert_close(out[vm], eager[vm], rtol=1e-12, atol=1e-12)
    assert torch.all(out[~vm] == 0) and torch.all(lse[~valid[:, None, :].expand_as(lse)] == 0)


def test_chunked_forward_packed_equals_padded():
    lens = [5, 1, 12]
    q, k, v, feats, w, b, seqlens = _padded_case(3, 12, 2, 16, 16, 22, lens=lens)
    out_p, lse_p = oracle.attention_fp64_chunked(q, k, v, feats, w, b, seqlens)
    pack = lambda x: torch.cat([x[i, :, :n].transpose(0, 1) for i, n in enumerate(lens)], 0)
    fpack = torch.cat([feats[i, :n] for i, n in enumerate(lens)], 0)
    cu = torch.tensor([0, 5, 6, 18])
    out_v, lse_v = oracle.attention_fp64_chunked(pack(q), pack(k), pack(v), fpack, w, b,
                                                 cu_seqlens=cu, row_block=4)
    torch.testing.assert_close(out_v, pack(out_p), rtol=1e-13, atol=1e-13)
    torch.testing.assert_close(lse_v, pack(lse_p[..., None])[..., 0], rtol=1e-13, atol=1e-13)


@pytest.mark.parametrize("flags", FLAGS)
def test_chunked_backward_matches_autograd(flags):
    q, k, v, feats, w, b, seqlens = _padded_case(2, 13, 2, 8, 6, 31, lens=[13, 4])
    valid = oracle.valid_row_mask(2, 13, seqlens)
    mask = oracle.float_padding_mask(valid, torch.float64)
    g = torch.randn(q.shape, dtype=torch.float64, generator=torch.Generator().manual_seed(2))
    leaves = [t.clone().requires_grad_(True) for t in (q, k, v, w, b)]
    out = oracle.attention(leaves[0], leaves[1], leaves[2], feats, leaves[3], leaves[4],
                           key_padding_mask=mask, use_attn_bias=flags[0],
                           use_activation_bias=flags[1])
    (out * g * valid[:, None, :, None]).sum().backward()
    got = oracle.backward_fp64_chunked(q, k, v, feats, w, b, g, seqlens,
                                       use_attn_bias=flags[0], use_activation_bias=flags[1],
                                       row_block=3, return_rowsum=True)
    for name, mine, leaf in zip("q k v W b".split(), got[:5], leaves):
        if name in ("W", "b") and not (flags[0] or flags[1]):
            assert mine is None and leaf.grad is None
            continue
        torch.testing.assert_close(mine, leaf.grad, rtol=1e-10, atol=1e-10, msg=name)
    assert got[5].abs().max() < 1e-12  # rowsum(dS) == 0


def test_eager_oracle_gradcheck():
    q, k, v, feats, w, b, _ = _padded_case(1, 4, 2, 4, 6, 41)
    feats = feats * 0.3
    fn = lambda q_, k_, v_, w_, b_: oracle.attention(q_, k_, v_, feats, w_, b_)
    args = [t.clone().requires_grad_(True) for t in (q, k, v, w, b)]
    assert torch.autograd.gradcheck(fn, args, eps=1e-6, atol=1e-6)


@pytest.mark.parametrize("flags", FLAGS[:3])
def test_backward_closed_forms_single_token(flags):
    q, k, v, feats, w, b, seqlens = _padded_case(2, 1, 3, 16, 16, 51)
    g = torch.randn(q.shape, dtype=torch.float64)
    dq, dk, dv, dW, db = oracle.backward_fp64_chunked(
        q, k, v, feats, w, b, g, seqlens, use_attn_bias=flags[0], use_activation_bias=flags[1])
    assert dq.abs().max() < 1e-14 and dk.abs().max() < 1e-14
    torch.testing.assert_close(dv, g, rtol=0, atol=1e-14)
    if flags[1]:
        torch.testing.assert_close(db, g.sum((0, 1, 2)), rtol=1e-12, atol=1e-12)
    else:
        assert db.abs().max() < 1e-12  # logit-only db vanishes (softmax shift)


@pytest.mark.parametrize("flags", FLAGS)
def test_event_rows_blocks_sum_to_whole_event(flags):
    """The row-block evaluator, summed over blocks, equals the whole-event
    chunked forward and backward (out, lse, dq, rowsum row by row; dk, dv, dW,
    db as the sum of the blocks' contributions)."""
    n = 19
    q, k, v, feats, w, b, seqlens = _padded_case(1, n, 3, 16, 8, 61)
    g = torch.randn(q.shape, dtype=torch.float64, generator=torch.Generator().manual_seed(5))
    kw = dict(use_attn_bias=flags[0], use_activation_bias=flags[1])
    out, lse = oracle.attention_fp64_chunked(q, k, v, feats, w, b, seqlens, **kw)
    dq, dk, dv, dW, db, rs = oracle.backward_fp64_chunked(q, k, v, feats, w, b, g, seqlens, return_rowsum=True,
                                                          **kw)
    acc = {"dk": 0, "dv": 0, "dW": 0, "db": 0}
    for r0, r1 in ((0, 7), (7, 8), (8, 19)):
        blk = oracle.event_rows_fp64(q[0], k[0], v[0], feats[0], w, b, g[0], (r0, r1), **kw)
        torch.testing.assert_close(blk["out"], out[0, :, r0:r1], rtol=1e-12, atol=1e-12)
        torch.testing.assert_close(blk["lse"], lse[0, :, r0:r1], rtol=1e-12, atol=1e-12)
        torch.testing.assert_close(blk["dq"], dq[0, :, r0:r1], rtol=1e-11, atol=1e-11)
        torch.testing.assert_close(blk["rowsum"], rs[0, :, r0:r1], rtol=0, atol=1e-12)
        for name in acc:
            if blk[name] is not None:
                acc[name] = acc[name] + blk[name]
    torch.testing.assert_close(acc["dk"], dk[0], rtol=1e-11, atol=1e-11)
    torch.testing.assert_close(acc["dv"], dv[0], rtol=1e-11, atol=1e-11)
    if flags[0] or flags[1]:
        torch.testing.assert_close(acc["dW"], dW, rtol=1e-11, atol=1e-11)
        torch.testing.assert_close(acc["db"], db, rtol=1e-11, atol=1e-11)


def test_event_rows_block_is_the_masked_upstream_gradient():
    """A block's gradient contributions are the gradients of the whole event
    under an upstream gradient that is zero outside the block (autograd
    through the eager restatement)."""
    n, r0, r1 = 11, 3, 8
    q, k, v, feats, w, b, _ = _padded_case(1, n, 2, 8, 6, 71)
    g = torch.randn(q.shape, dtype=torch.float64, generator=torch.Generator().manual_seed(6))
    g[:, :, :r0] = 0
    g[:, :, r1:] = 0
    leaves = [t.clone().requires_grad_(True) for t in (q, k, v, w, b)]
    out = oracle.attention(leaves[0], leaves[1], leaves[2], feats, leaves[3], leaves[4])
    (out * g).sum().backward()
    blk = oracle.event_rows_fp64(q[0], k[0], v[0], feats[0], w, b, g[0], (r0, r1))
    torch.testing.assert_close(blk["dq"], leaves[0].grad[0, :, r0:r1], rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(blk["dk"], leaves[1].grad[0], rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(blk["dv"], leaves[2].grad[0], rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(blk["dW"], leaves[3].grad, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(blk["db"], leaves[4].grad, rtol=1e-10, atol=1e-10)


def test_event_rows_in_float32_is_the_eager_definition():
    """The float32 row-block evaluation equals the eager restatement run in
    float32 (the 2x-eager yardstick) on the block's rows."""
    n, r0, r1 = 21, 4, 15
    q, k, v, feats, w, b, _ = _padded_case(1, n, 2, 16, 8, 81)
    g = torch.randn(q.shape, dtype=torch.float64, generator=torch.Generator().manual_seed(8))
    g[:, :, :r0] = 0
    g[:, :, r1:] = 0
    f32 = lambda t: t.float()
    leaves = [f32(t).clone().requires_grad_(True) for t in (q, k, v, w, b)]
    out = oracle.attention(leaves[0], leaves[1], leaves[2], f32(feats), leaves[3], leaves[4])
    (out * f32(g)).sum().backward()
    blk = oracle.event_rows_fp64(q[0], k[0], v[0], feats[0], w, b, g[0], (r0, r1), dtype=torch.float32)
    assert blk["out"].dtype == torch.float32
    torch.testing.assert_close(blk["out"], out[0, :, r0:r1].detach(), rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(blk["dq"], leaves[0].grad[0, :, r0:r1], rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(blk["dk"], leaves[1].grad[0], rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(blk["dv"], leaves[2].grad[0], rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(blk["dW"], leaves[3].grad, rtol=1e-4, atol=1e-4)


# ------------------------------------------- planted mistakes must be caught


def test_planted_sin_cos_swap_is_caught(monkeypatch):
    def swapped(x, c):
        theta = x.unsqueeze(-1) * oracle.frequencies(c).to(x.device)
        return torch.cat((torch.cos(theta), torch.sin(theta)), dim=-1)

    monkeypatch.setattr(spec, "embed_angle", swapped)
    with pytest.raises(AssertionError):
        test_pair_features_match_reference_vectors("n16", "f64")
    with pytest.raises(AssertionError):
        test_single_token_event_closed_form(16)


def test_planted_time_sign_is_caught(monkeypatch):
    def wrong(rows, cols):
        spatial = (rows[:, :, None, :3] - cols[:, None, :, :3]).pow(2).sum(-1)
        temporal = ((rows[:, :, None, 3] - cols[:, None, :, 3]) * spec.TIME_SCALE).pow(2)
        interval = spatial + temporal  # wrong metric signature
        signed = torch.sign(interval) * torch.sqrt(torch.abs(interval))
        return spec.SINEMB_INPUT_SCALE * signed.clip(-spec.SINEMB_CLIP, spec.SINEMB_CLIP)

    monkeypatch.setattr(spec, "pair_angle_rect", wrong)
    with pytest.raises(AssertionError):
        test_embedding_bruteforce_scalar()
    with pytest.raises(AssertionError):
        test_pair_features_match_reference_vectors("n16", "f64")


def test_planted_weight_transpose_is_caught(monkeypatch):
    orig = spec.pair_features
    monkeypatch.setattr(spec, "pair_features", lambda f, w, b: orig(f, w.t().contiguous(), b))
    with pytest.raises(AssertionError):
        test_attention_matches_reference_vectors("n16", "f64", (True, True))


def test_planted_unnormalised_rowsum_is_caught(monkeypatch):
    orig_softmax = torch.softmax
    monkeypatch.setattr(spec.torch, "softmax", lambda x, dim: orig_softmax(x, dim) * 1.01)
    with pytest.raises(AssertionError):
        test_chunked_backward_matches_autograd((True, True))
