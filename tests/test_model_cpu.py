"""The model-side module's projections, on the CPU (no kernel calls).

`SpacetimeAttention.project_qkv` (one fused GEMM for self-attention) must
give the values of the reference's `attention_rel_oracle_inputs` (separate
linears, then `split_heads`, reference.py:198-223) and carry the same
gradients back to x and the weights.
"""

import pytest
import torch

from flash_spacetime_amd import SpacetimeAttention, attention_rel_oracle_inputs
from flash_spacetime_amd.forward import is_token_major


def _module(qkv_bias: bool) -> SpacetimeAttention:
    torch.manual_seed(0)
    m = SpacetimeAttention(96, num_heads=3, channels=16, qkv_bias=qkv_bias, dtype=torch.float64)
    if qkv_bias:
        with torch.no_grad():
            m.q_bias.normal_()
            m.v_bias.normal_()
    return m


@pytest.mark.parametrize("qkv_bias", [False, True])
@pytest.mark.parametrize("cross", [False, True], ids=["self", "cross"])
def test_project_qkv_matches_attention_rel_inputs(qkv_bias, cross):
    m = _module(qkv_bias)
    gen = torch.Generator().manual_seed(1)
    x = torch.randn(2, 7, 96, generator=gen, dtype=torch.float64, requires_grad=True)
    kv = torch.randn(2, 7, 96, generator=gen, dtype=torch.float64, requires_grad=True) if cross else None
    got = m.project_qkv(x, kv)
    want = attention_rel_oracle_inputs(m, x, kv)
    for a, b in zip(got, want):
        assert a.shape == (2, 3, 7, 32)
        # self-attention: slots of one [B, L, 3, H, D] projection (token
        # stride 3 H D); cross-attention: token-major views of three linears
        assert a.stride(2) == 3 * 96 if not cross else is_token_major(a)
        torch.testing.assert_close(a, b, rtol=1e-13, atol=1e-13)
    gw = [torch.randn(a.shape, generator=gen, dtype=torch.float64) for a in got]
    params = [x] + ([kv] if cross else []) + [p for p in (m.proj_q.weight, m.proj_k.weight, m.proj_v.weight,
                                                           m.q_bias, m.v_bias) if p is not None]
    g_got = torch.autograd.grad(sum((a * g).sum() for a, g in zip(got, gw)), params)
    g_want = torch.autograd.grad(sum((a * g).sum() for a, g in zip(want, gw)), params)
    for a, b in zip(g_got, g_want):
        torch.testing.assert_close(a, b, rtol=1e-12, atol=1e-12)


def test_module_parameters_follow_attention_rel():
    m = _module(True)
    names = {n for n, _ in m.named_parameters()}
    assert {"proj_q.weight", "proj_k.weight", "proj_v.weight", "q_bias", "v_bias", "proj.weight",
            "proj.bias", "rel_proj.weight", "rel_proj.bias"} == names
    assert m.rel_proj.weight.shape == (32, 16) and m.num_heads == 3
    assert _module(False).q_bias is None


def test_backward_refuses_gradient_buffers_of_another_layout():
    """Regression: the kernels address dq, dk, dv exactly as q, k, v. With
    interleaved operands, `empty_like` of a slot view is contiguous and would
    be written past its end, so the host layer must refuse it (and any
    mismatched buffer) before launching anything."""
    from flash_spacetime_amd import _lib
    from flash_spacetime_amd.backward import _run_backward
    from flash_spacetime_amd.forward import _qkv_views

    B, L, H, D, C = 2, 5, 3, 32, 16
    qkv = torch.zeros(B, L, 3, H, D)
    q, k, v = _qkv_views(qkv, False)
    dims = (_lib.FST_F32, 3 | _lib.FST_TOKEN_MAJOR | _lib.FST_QKV_INTERLEAVED, B, H, L, 0, D, C)
    lse = torch.zeros(B, L, H).transpose(1, 2)
    do = torch.zeros(B, L, H, D).transpose(1, 2)
    with pytest.raises(ValueError, match="interleaved"):
        _run_backward(dims, q, k, v, None, None, None, None, lse, do, 1.0, (B, H, L))


def test_backward_refuses_lse_of_another_shape():
    """The kernels read lse at every (row, head) of the operands: a smaller
    lse is refused before any launch (as is one of another dtype)."""
    from flash_spacetime_amd import _lib
    from flash_spacetime_amd.backward import _run_backward

    B, L, H, D, C = 2, 5, 3, 32, 16
    q = torch.zeros(B, H, L, D)
    dims = (_lib.FST_F32, 3, B, H, L, 0, D, C)
    do = torch.zeros(B, H, L, D)
    for lse in (torch.zeros(B, H, L - 1), torch.zeros(B, H, L, dtype=torch.float64)):
        with pytest.raises(ValueError, match="lse"):
            _run_backward(dims, q, q, q, None, None, None, None, lse, do, 1.0, (B, H, L))
