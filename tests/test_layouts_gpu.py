"""GPU tests of the input formats and layouts the build adds to the reference's API.

* `torch.nested` jagged q / k / v (and feats) for the packed operator: the
  result and every gradient are bitwise those of the dense packed call on the
  same values and offsets.
* Padding masks whose valid tokens are not a prefix of each event (the
  reference accepts front-packed lengths only): valid rows and all gradients
  against the float64 oracle evaluated with the same mask (`pair_mask`, the
  spec's one-sided key mask), padding rows exactly zero.
* Heads-first views of token-major `[B, L, H, D]` memory (what `split_heads`
  makes of a projection) are read in place: results bitwise those of the
  contiguous call, returned as the same kind of view.
* One interleaved q/k/v tensor (`flash_spacetime_attention_qkv`, the output
  of a fused projection, padded `[B, L, 3, H, D]` or packed `[T, 3, H, D]`):
  output and the one gradient tensor bitwise those of the op on the split
  heads.
"""

import pytest
import torch

import oracle
from tests._cases import FLAGS, make_packed, make_padded, rel_err, seed_of

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from flash_spacetime_amd import flash_spacetime_attention, flash_spacetime_attention_varlen


def _holey_mask(batch: int, length: int, seed: int) -> torch.Tensor:
    """[B, L] validity with holes: ~60 % valid, every event non-empty, one
    event fully valid and one with a single valid token in the middle."""
    gen = torch.Generator().manual_seed(seed)
    valid = torch.rand(batch, length, generator=gen) < 0.6
    valid[:, length // 2] = True
    valid[0] = True
    if batch > 1:
        valid[-1] = False
        valid[-1, length // 3] = True
    return valid


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("flags", FLAGS[:3], ids=["attn1act1", "attn1act0", "attn0act1"])
def test_holey_mask_matches_oracle(dtype, flags):
    shape = (3, 70, 4, 32, 16)
    case = make_padded(*shape, seed=seed_of("holes", dtype, flags), masked=False)
    valid = _holey_mask(shape[0], shape[1], seed_of("holes-mask", dtype, flags))
    # The reference is evaluated on the dtype-rounded inputs, which isolates
    # the kernel's own error from input quantisation.
    for key in ("q", "k", "v", "weight", "bias"):
        case[key] = case[key].to(dtype).double()
    names = {"q": "q", "k": "k", "v": "v", "W": "weight", "b": "bias"}
    dev = "cuda"
    leaves = {n: case[c].to(dev, dtype).requires_grad_(True) for n, c in names.items()}
    out = flash_spacetime_attention(
        leaves["q"], leaves["k"], leaves["v"], case["feats"].to(dev), leaves["W"], leaves["b"],
        key_padding_mask=~valid.to(dev), use_attn_bias=flags[0], use_activation_bias=flags[1],
    )
    vm = valid[:, None, :, None].expand(out.shape)
    gw = torch.randn(out.shape, dtype=torch.float64, generator=torch.Generator().manual_seed(3)) * vm
    (out.double() * gw.to(dev)).sum().backward()

    ref_leaves = {n: case[c].clone().requires_grad_(True) for n, c in names.items()}
    ref = oracle.attention(
        ref_leaves["q"], ref_leaves["k"], ref_leaves["v"], case["feats"], ref_leaves["W"], ref_leaves["b"],
        key_padding_mask=oracle.float_padding_mask(valid, torch.float64),
        use_attn_bias=flags[0], use_activation_bias=flags[1],
    )
    (ref * gw).sum().backward()

    got = out.detach().cpu()
    assert (got[~vm] == 0).all(), "padding rows must be exactly zero"
    tol = 2e-2 if dtype == torch.bfloat16 else 1e-4
    err = rel_err(got * vm, ref.detach() * vm)
    assert err <= tol, f"output: relative error {err:.3e}"
    # fp32 gradients: 1e-3, the bound the fp32 large-logit test also uses
    # (sums over the event of E-weighted terms).
    gtol = 2e-2 if dtype == torch.bfloat16 else 1e-3
    keys = ["q", "k", "v"] + (["W"] if (flags[0] or flags[1]) else []) + (["b"] if flags[1] else [])
    if flags[0] and not flags[1]:
        # b enters only through the row-constant logit term qt.b: db = 0
        # (backward.py:616-622); the float64 oracle's value is rounding noise.
        assert leaves["b"].grad is None or (leaves["b"].grad == 0).all()
        assert ref_leaves["b"].grad.abs().max().item() < 1e-9
    for key in keys:
        g = leaves[key].grad
        assert g is not None and torch.isfinite(g).all(), key
        err = rel_err(g, ref_leaves[key].grad)
        assert err <= gtol, f"grad {key}: relative error {err:.3e}"


def test_front_packed_mask_keeps_the_lengths_path():
    """A front-packed mask and its lengths give bitwise the same result; a mask
    with holes agrees with the same events packed by hand."""
    shape = (3, 40, 4, 32, 16)
    case = make_padded(*shape, seed=seed_of("mask-paths"))
    dev = "cuda"
    g = {k: case[k].to(dev, torch.bfloat16) for k in ("q", "k", "v", "weight", "bias")}
    feats = case["feats"].to(dev)
    valid = oracle.valid_row_mask(3, 40, case["seqlens"]).to(dev)
    base = flash_spacetime_attention(g["q"], g["k"], g["v"], feats, g["weight"], g["bias"],
                                     case["seqlens"].to(dev))
    by_mask = flash_spacetime_attention(g["q"], g["k"], g["v"], feats, g["weight"], g["bias"],
                                        key_padding_mask=~valid)
    assert torch.equal(base, by_mask)

    holey = _holey_mask(3, 40, seed_of("mask-paths-holes")).to(dev)
    out = flash_spacetime_attention(g["q"], g["k"], g["v"], feats, g["weight"], g["bias"],
                                    key_padding_mask=~holey)
    counts = holey.sum(1).tolist()
    cu = torch.tensor([0] + torch.tensor(counts).cumsum(0).tolist(), dtype=torch.int32, device=dev)
    rows = lambda x: x.transpose(1, 2)[holey]
    packed = flash_spacetime_attention_varlen(rows(g["q"]), rows(g["k"]), rows(g["v"]), feats[holey],
                                              g["weight"], g["bias"], cu)
    assert torch.equal(out.transpose(1, 2)[holey], packed)
    assert (out.transpose(1, 2)[~holey] == 0).all()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_nested_inputs_match_dense_packed(dtype):
    lengths = [17, 64, 1, 200, 33]
    case = make_packed(lengths, 4, 32, 16, seed_of("nested", dtype))
    dev = "cuda"
    cu = case["cu"].to(dev)
    gw = torch.randn(case["q"].shape, generator=torch.Generator().manual_seed(5)).to(dev, dtype)

    def run(nested: bool):
        leaves = {k: case[k].to(dev, dtype).requires_grad_(True) for k in ("q", "k", "v")}
        w = case["weight"].to(dev, dtype).requires_grad_(True)
        b = case["bias"].to(dev, dtype).requires_grad_(True)
        feats = case["feats"].to(dev)
        if nested:
            offs = cu.long()
            nt = {k: torch.nested.nested_tensor_from_jagged(x, offs) for k, x in leaves.items()}
            fnt = torch.nested.nested_tensor_from_jagged(feats, offs)
            out_nt = flash_spacetime_attention_varlen(nt["q"], nt["k"], nt["v"], fnt, w, b)
            assert out_nt.is_nested and torch.equal(out_nt.offsets(), offs)
            out = out_nt.values()
        else:
            out = flash_spacetime_attention_varlen(leaves["q"], leaves["k"], leaves["v"], feats, w, b, cu)
        (out.float() * gw.float()).sum().backward()
        return out.detach(), [leaves[k].grad for k in ("q", "k", "v")] + [w.grad, b.grad]

    out_d, grads_d = run(False)
    out_n, grads_n = run(True)
    assert torch.equal(out_d, out_n)
    for a, b in zip(grads_d, grads_n):
        assert torch.equal(a, b)


def _token_major(x: torch.Tensor) -> torch.Tensor:
    """The same values as a heads-first view of [B, L, H, D] memory."""
    return x.transpose(1, 2).contiguous().transpose(1, 2)


# (dtype, shape): bf16 tile kernels, the bf16 layout on the fallback backward
# (H=16, D=C=64), fp32 kernels; fp32 has no backward at H=16, D=C=64.
_TM_CASES = [(torch.bfloat16, (3, 50, 12, 32, 16)), (torch.bfloat16, (2, 40, 16, 64, 64)),
             (torch.bfloat16, (2, 33, 5, 48, 32)), (torch.float32, (3, 50, 12, 32, 16)),
             (torch.float32, (2, 40, 8, 64, 64)), (torch.float32, (2, 33, 5, 48, 32))]


@pytest.mark.parametrize("dtype,shape", _TM_CASES,
                         ids=[f"{str(d)[6:]}-{'x'.join(map(str, s))}" for d, s in _TM_CASES])
@pytest.mark.parametrize("flags", FLAGS[:3], ids=["attn1act1", "attn1act0", "attn0act1"])
def test_token_major_views_match_contiguous(dtype, shape, flags):
    """Heads-first views of [B, L, H, D] memory (split_heads of a projection)
    are read in place: output, lse and every gradient are bitwise those of
    the contiguous [B, H, L, D] call, and come back as the same kind of view."""
    case = make_padded(*shape, seed=seed_of("token-major", dtype, shape, flags))
    dev = "cuda"
    seqlens = case["seqlens"].to(dev)
    feats = case["feats"].to(dev)
    gw = torch.randn(shape[0], shape[2], shape[1], shape[3], generator=torch.Generator().manual_seed(9))

    def run(token_major: bool):
        conv = _token_major if token_major else (lambda x: x.contiguous())
        leaves = {k: conv(case[k].to(dev, dtype)).requires_grad_(True) for k in ("q", "k", "v")}
        w = case["weight"].to(dev, dtype).requires_grad_(True)
        b = case["bias"].to(dev, dtype).requires_grad_(True)
        out = flash_spacetime_attention(leaves["q"], leaves["k"], leaves["v"], feats, w, b, seqlens,
                                        use_attn_bias=flags[0], use_activation_bias=flags[1])
        (out.float() * conv(gw.to(dev))).sum().backward()
        return out.detach(), [leaves[k].grad for k in ("q", "k", "v")] + [w.grad, b.grad]

    out_c, grads_c = run(False)
    out_t, grads_t = run(True)
    assert out_t.transpose(1, 2).is_contiguous() and not out_t.is_contiguous()
    assert torch.equal(out_c, out_t)
    for a, b in zip(grads_c, grads_t):
        assert (a is None) == (b is None)
        if a is not None:
            assert torch.equal(a, b)
    for g in grads_t[:3]:
        assert g.transpose(1, 2).is_contiguous()


def test_token_major_launcher_lse_and_rowsum():
    """flash_spacetime_forward / _backward with token-major operands: lse comes
    back as a heads-first view with the contiguous call's values; a
    contiguous rowsum buffer and a contiguous grad_out are accepted."""
    from flash_spacetime_amd import flash_spacetime_backward, flash_spacetime_forward

    shape = (3, 45, 8, 32, 16)
    case = make_padded(*shape, seed=seed_of("token-major-launcher"))
    dev, dt = "cuda", torch.bfloat16
    q, k, v = (case[n].to(dev, dt) for n in ("q", "k", "v"))
    feats, w, b = case["feats"].to(dev), case["weight"].to(dev), case["bias"].to(dev)
    sl = case["seqlens"].to(dev)
    do = torch.randn(q.shape, generator=torch.Generator().manual_seed(4)).to(dev, dt)
    o_c, lse_c = flash_spacetime_forward(q, k, v, feats, w, b, sl)
    tq, tk, tv = (_token_major(x) for x in (q, k, v))
    o_t, lse_t = flash_spacetime_forward(tq, tk, tv, feats, w, b, sl)
    assert torch.equal(o_c, o_t) and torch.equal(lse_c, lse_t)
    assert lse_t.transpose(1, 2).is_contiguous()
    rs_c = torch.full(lse_c.shape, float("nan"), device=dev)
    rs_t = torch.full(lse_c.shape, float("nan"), device=dev)
    g_c = flash_spacetime_backward(q, k, v, feats, w, b, sl, lse_c, do, rowsum=rs_c)
    # The token-major call gets lse contiguous and grad_out contiguous: both
    # are brought into the operands' layout.
    g_t = flash_spacetime_backward(tq, tk, tv, feats, w, b, sl, lse_c, do, rowsum=rs_t)
    for a, c in zip(g_c, g_t):
        assert torch.equal(a, c)
    assert torch.equal(rs_c, rs_t)


def test_token_major_with_holey_mask_and_mixed_layouts():
    """A mask with holes on token-major views matches the contiguous call; q
    token-major with k, v contiguous takes the contiguous path."""
    shape = (3, 40, 4, 32, 16)
    case = make_padded(*shape, seed=seed_of("token-major-mixed"), masked=False)
    dev, dt = "cuda", torch.bfloat16
    q, k, v = (case[n].to(dev, dt) for n in ("q", "k", "v"))
    feats, w, b = case["feats"].to(dev), case["weight"].to(dev), case["bias"].to(dev)
    holey = _holey_mask(3, 40, seed_of("token-major-holes")).to(dev)
    base = flash_spacetime_attention(q, k, v, feats, w, b, key_padding_mask=~holey)
    tm = flash_spacetime_attention(_token_major(q), _token_major(k), _token_major(v), feats, w, b,
                                   key_padding_mask=~holey)
    assert torch.equal(base, tm) and tm.transpose(1, 2).is_contiguous()
    sl = case["seqlens"].to(dev)
    mixed = flash_spacetime_attention(_token_major(q), k, v, feats, w, b, sl)
    assert torch.equal(mixed, flash_spacetime_attention(q, k, v, feats, w, b, sl))


_QKV_CASES = [(torch.bfloat16, (3, 50, 12, 32, 16)), (torch.bfloat16, (2, 40, 16, 64, 64)),
              (torch.float32, (3, 50, 12, 32, 16)), (torch.float32, (2, 33, 5, 48, 32))]


@pytest.mark.parametrize("dtype,shape", _QKV_CASES,
                         ids=[f"{str(d)[6:]}-{'x'.join(map(str, s))}" for d, s in _QKV_CASES])
@pytest.mark.parametrize("flags", FLAGS[:3], ids=["attn1act1", "attn1act0", "attn0act1"])
def test_qkv_interleaved_matches_split_heads(dtype, shape, flags):
    """flash_spacetime_attention_qkv on one [B, L, 3, H, D] tensor: output and
    the gradient tensor bitwise those of flash_spacetime_attention on the
    contiguous split heads (dq, dk, dv stacked into the same layout)."""
    from flash_spacetime_amd import flash_spacetime_attention_qkv

    bsz, length, heads, dim, _ = shape
    case = make_padded(*shape, seed=seed_of("qkv", dtype, shape, flags))
    dev = "cuda"
    seqlens, feats = case["seqlens"].to(dev), case["feats"].to(dev)
    qkv0 = torch.stack([case[n].transpose(1, 2) for n in ("q", "k", "v")], 2).to(dev, dtype).contiguous()
    gw = torch.randn(bsz, length, heads, dim, generator=torch.Generator().manual_seed(11)).to(dev)
    w0, b0 = case["weight"].to(dev, dtype), case["bias"].to(dev, dtype)

    qkv = qkv0.clone().requires_grad_(True)
    w, b = w0.clone().requires_grad_(True), b0.clone().requires_grad_(True)
    out = flash_spacetime_attention_qkv(qkv, feats, w, b, seqlens, use_attn_bias=flags[0],
                                        use_activation_bias=flags[1])
    assert out.shape == (bsz, length, heads, dim) and out.is_contiguous()
    (out.float() * gw).sum().backward()

    leaves = [qkv0[:, :, i].transpose(1, 2).contiguous().requires_grad_(True) for i in range(3)]
    w2, b2 = w0.clone().requires_grad_(True), b0.clone().requires_grad_(True)
    ref = flash_spacetime_attention(*leaves, feats, w2, b2, seqlens, use_attn_bias=flags[0],
                                    use_activation_bias=flags[1])
    (ref.float() * gw.transpose(1, 2)).sum().backward()

    assert torch.equal(out, ref.transpose(1, 2))
    assert torch.equal(qkv.grad, torch.stack([t.grad.transpose(1, 2) for t in leaves], 2))
    for a, c in ((w.grad, w2.grad), (b.grad, b2.grad)):
        assert (a is None) == (c is None) and (a is None or torch.equal(a, c))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_qkv_interleaved_packed_and_masks(dtype):
    """Packed [T, 3, H, D] with cu_seqlens against the varlen op on q, k, v;
    a padded qkv with a mask with holes against the split-heads op with the
    same mask (both bitwise, gradients included)."""
    from flash_spacetime_amd import flash_spacetime_attention_qkv

    dev = "cuda"
    lengths = [17, 64, 1, 120, 33]
    case = make_packed(lengths, 6, 32, 16, seed_of("qkv-packed", dtype))
    cu, feats = case["cu"].to(dev), case["feats"].to(dev)
    w, b = case["weight"].to(dev, dtype), case["bias"].to(dev, dtype)
    qkv0 = torch.stack([case[n] for n in ("q", "k", "v")], 1).to(dev, dtype).contiguous()
    gw = torch.randn(qkv0.shape[0], 6, 32, generator=torch.Generator().manual_seed(12)).to(dev)
    qkv = qkv0.clone().requires_grad_(True)
    out = flash_spacetime_attention_qkv(qkv, feats, w, b, cu_seqlens=cu)
    (out.float() * gw).sum().backward()
    leaves = [qkv0[:, i].contiguous().requires_grad_(True) for i in range(3)]
    ref = flash_spacetime_attention_varlen(*leaves, feats, w, b, cu)
    (ref.float() * gw).sum().backward()
    assert torch.equal(out, ref)
    assert torch.equal(qkv.grad, torch.stack([t.grad for t in leaves], 1))

    shape = (3, 40, 4, 32, 16)
    pc = make_padded(*shape, seed=seed_of("qkv-holes", dtype), masked=False)
    holey = _holey_mask(3, 40, seed_of("qkv-holes-mask", dtype)).to(dev)
    feats = pc["feats"].to(dev)
    w, b = pc["weight"].to(dev, dtype), pc["bias"].to(dev, dtype)
    qkv0 = torch.stack([pc[n].transpose(1, 2) for n in ("q", "k", "v")], 2).to(dev, dtype).contiguous()
    qkv = qkv0.clone().requires_grad_(True)
    out = flash_spacetime_attention_qkv(qkv, feats, w, b, key_padding_mask=~holey)
    gw = torch.randn(out.shape, generator=torch.Generator().manual_seed(13)).to(dev)
    (out.float() * gw).sum().backward()
    leaves = [qkv0[:, :, i].transpose(1, 2).contiguous().requires_grad_(True) for i in range(3)]
    ref = flash_spacetime_attention(*leaves, feats, w, b, key_padding_mask=~holey)
    (ref.float() * gw.transpose(1, 2)).sum().backward()
    assert torch.equal(out, ref.transpose(1, 2))
    assert torch.equal(qkv.grad, torch.stack([t.grad.transpose(1, 2) for t in leaves], 2))
