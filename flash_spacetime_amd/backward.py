"""Deterministic fused backward of spacetime-bias attention.

Mirrors the reference launcher `flash_spacetime_backward`
(src/flash_spacetime/backward.py:488-630): same arguments and return
value `(dq, dk, dv, dW, db)`. The host prologue (u, w~ = dO W, dO.b), both
kernels and the host epilogue (dq projection, dW, db) run inside the HIP
library; the softmax row term is formed in-kernel as
D = sum(p * dp) / sum(p) from the very p and dp that build dS, so
rowsum(dS) vanishes by construction (backward.py:23-32, 371-377).
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import Tensor

from . import _lib, tune
from .forward import _Prepared, _bf16, _vec_in_layout, head_groups


def _same_layout(a: Tensor, b: Tensor) -> bool:
    return all(sa == sb for sa, sb, n in zip(a.stride(), b.stride(), a.shape) if n > 1)


def _run_backward(dims, q, k, v, pos4, w32, b32, lens, lse, grad_out, scale, vec_shape,
                  rowsum: Optional[Tensor] = None, out_like: Optional[Tensor] = None,
                  grads: Optional[Tuple[Tensor, Tensor, Tensor]] = None, out: Optional[Tensor] = None):
    """Launch the backward. grad_out is brought into the layout of `out_like`
    (default q: contiguous, or token-major when the flags say so; empty_like
    keeps a dense view's strides); dq, dk, dv are written into `grads` when
    given (the slots of one interleaved gradient tensor), else into tensors
    laid out like q, k, v. `out`, the forward's output, is handed to the
    kernels where it has grad_out's final shape, dtype and layout (the bf16
    rows kernel takes its reference D from it); otherwise it is left out,
    which changes nothing but the kernel's schedule of D updates."""
    if grad_out.shape != q.shape:
        raise ValueError(f"grad_out must have the shape of the output {tuple(q.shape)}")
    interleaved = bool(dims[1] & _lib.FST_QKV_INTERLEAVED)
    if interleaved and (grads is None or out_like is None):
        # empty_like of a slot view of [.., 3, H, D] is contiguous, not
        # interleaved: the kernels would write past its end.
        raise ValueError("interleaved q / k / v need the gradient slots of one tensor and the output layout")
    token_major = bool(dims[1] & (_lib.FST_TOKEN_MAJOR | _lib.FST_PACKED))
    if (tuple(lse.shape) != tuple(vec_shape) or lse.dtype != torch.float32 or lse.device != q.device
            or not (lse.transpose(1, 2).is_contiguous() if token_major and lse.dim() == 3 else lse.is_contiguous())):
        raise ValueError(f"lse must be float32 {tuple(vec_shape)} on the operands' device, laid out as they are")
    if rowsum is not None and (rowsum.shape != lse.shape or rowsum.dtype != torch.float32
                               or rowsum.device != q.device):
        raise ValueError(f"rowsum must be float32 of the shape of lse {tuple(lse.shape)} on the operands' device")
    lib = _lib.load()
    _lib.require_gpu(grad_out)
    groups = head_groups(dims[0], dims[3], dims[6], dims[7])
    if len(groups) > 1:
        return _run_backward_grouped(groups, dims, q, k, v, pos4, w32, b32, lens, lse, grad_out, scale,
                                     rowsum, grads, out)
    like = q if out_like is None else out_like
    do = grad_out.to(q.dtype)
    if not _same_layout(do, like):
        do = torch.empty_like(like).copy_(do)
    if out is not None and not (out.shape == do.shape and out.dtype == do.dtype and out.device == do.device
                                and _same_layout(out, do)):
        out = None
    if grads is not None:
        dq, dk, dv = grads
    else:
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    # The kernels address dq, dk, dv exactly as q, k, v (and rowsum as lse):
    # buffers of another layout or shape are refused rather than overrun.
    for name, gb, src in (("dq", dq, q), ("dk", dk, k), ("dv", dv, v)):
        if gb.shape != src.shape or gb.dtype != src.dtype or not _same_layout(gb, src):
            raise ValueError(f"{name} buffer must have the shape, dtype and layout of its operand")
    rs = rowsum
    if rowsum is not None and not _same_layout(rowsum, lse):
        rs = torch.empty_like(lse)
    dw = torch.empty(w32.shape, device=q.device, dtype=torch.float32)
    db = torch.empty(q.shape[-1], device=q.device, dtype=torch.float32) if b32 is not None else None
    ws_bytes = lib.fst_backward_workspace_bytes(*dims)
    ws = torch.empty(max(ws_bytes, 1), device=q.device, dtype=torch.uint8)

    def run(phases: int, flags: int) -> int:
        return lib.fst_backward_phases(
            phases, dims[0], flags, *dims[2:],
            _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(pos4), _lib.ptr(w32), _lib.ptr(b32),
            _lib.ptr(lens), _lib.ptr(lse), _lib.ptr(do), _lib.ptr(out), scale,
            _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(dw), _lib.ptr(db), _lib.ptr(rs),
            _lib.ptr(ws), ws_bytes, _lib.stream_handle(q.device),
        )

    with torch.cuda.device(q.device):
        plan = tune.backward_plan(dims, run)
        rc = run(_lib.FST_BWD_ALL, dims[1] | plan)
    _lib.check(rc, "flash_spacetime_backward")
    if rs is not rowsum:
        rowsum.copy_(rs)
    return dq, dk, dv, dw, db


def _run_backward_grouped(groups, dims, q, k, v, pos4, w32, b32, lens, lse, grad_out, scale, rowsum, grads,
                          out=None):
    """The backward one head group at a time (head_groups): each group's
    operands as contiguous tensors, its gradients copied into the full ones,
    dW and db summed over the groups in order."""
    if grads is not None:
        dq, dk, dv = grads
    else:
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    do = grad_out.to(q.dtype)
    dw = torch.zeros(w32.shape, device=q.device, dtype=torch.float32)
    db = torch.zeros(q.shape[-1], device=q.device, dtype=torch.float32) if b32 is not None else None
    flags = dims[1] & ~(_lib.FST_TOKEN_MAJOR | _lib.FST_QKV_INTERLEAVED)
    for h0, h1 in groups:
        part = lambda t: t[:, h0:h1].contiguous()  # noqa: E731
        lse_g = part(lse)
        rs_g = torch.empty_like(lse_g) if rowsum is not None else None
        sub = (dims[0], flags, dims[2], h1 - h0) + tuple(dims[4:])
        g_dq, g_dk, g_dv, g_dw, g_db = _run_backward(sub, part(q), part(k), part(v), pos4, w32, b32, lens,
                                                     lse_g, part(do), scale, tuple(lse_g.shape), rowsum=rs_g,
                                                     out=None if out is None else part(out))
        dq[:, h0:h1].copy_(g_dq)
        dk[:, h0:h1].copy_(g_dk)
        dv[:, h0:h1].copy_(g_dv)
        dw += g_dw
        if db is not None:
            db += g_db
        if rowsum is not None:
            rowsum[:, h0:h1].copy_(rs_g)
    return dq, dk, dv, dw, db


def flash_spacetime_backward(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    feats: Tensor,
    weight: Tensor,
    bias: Optional[Tensor],
    seqlens: Optional[Tensor],
    lse: Tensor,
    grad_out: Tensor,
    scale: Optional[float] = None,
    use_attn_bias: bool = True,
    use_activation_bias: bool = True,
    block_m: Optional[int] = None,
    block_n: Optional[int] = None,
    num_warps: Optional[int] = None,
    num_stages: Optional[int] = None,
    cu_seqlens: Optional[Tensor] = None,
    rowsum: Optional[Tensor] = None,
    out: Optional[Tensor] = None,
) -> Tuple[Tensor, Tensor, Tensor, Tensor, Optional[Tensor]]:
    """Deterministic backward from the saved lse; returns (dq, dk, dv, dW, db).

    Gradients come back in the input dtypes (dW in the weight dtype, db in
    the bias dtype, or None without a bias). Upstream gradients on padding
    rows are ignored (backward.py:526-532). `rowsum`, if given (float32,
    shaped like lse), receives sum_j dS_ij per row and head. The reference's
    tile arguments select compiled kernel variants (tune.plan_from_tiles):
    block_m the float32 kernels' rows (keys) per workgroup, block_n their
    chunk, num_warps the bf16 rows kernel's waves per workgroup (4 or 8),
    each the nearest offered value; None (the default here; the reference
    defaults to 16, 16, 8) keeps the library's tuned or static choice, and
    num_stages is accepted with no counterpart (loads run one chunk ahead).
    `out` (optional, no reference counterpart) is the forward's output: with
    it the bf16 rows kernel forms dS against a reference D taken from it and
    corrects to its own D = sum P dP / sum P once, after the last key chunk;
    the gradients agree with those without it up to rounding.
    """
    del num_stages
    if q.dtype == torch.float16:  # the bf16 path, as the forward launcher runs it
        dq, dk, dv, dw, db = flash_spacetime_backward(
            *_bf16(q, k, v), feats, weight, bias, seqlens, lse, grad_out.to(torch.bfloat16), scale,
            use_attn_bias, use_activation_bias, block_m=block_m, block_n=block_n, num_warps=num_warps,
            cu_seqlens=cu_seqlens, rowsum=rowsum, out=None if out is None else out.to(torch.bfloat16))
        return dq.to(q.dtype), dk.to(q.dtype), dv.to(q.dtype), dw, db
    prep = _Prepared(q, k, v, feats, weight, bias, seqlens, scale, use_attn_bias,
                     use_activation_bias, cu_seqlens)
    with tune.tile_request(block_m, block_n, num_warps):
        dq, dk, dv, dw, db = _run_backward(
            prep.dims(), prep.q, prep.k, prep.v, prep.pos4, prep.weight, prep.bias, prep.lens,
            _vec_in_layout(lse, prep.token_major), grad_out, prep.scale, prep.vec_shape(), rowsum, out=out,
        )
    return (
        dq,
        dk,
        dv,
        dw.to(weight.dtype),
        db.to(bias.dtype) if (db is not None and bias is not None) else db,
    )
