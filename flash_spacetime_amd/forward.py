"""Fused spacetime-bias attention: public operators and the forward launcher.

Mirrors the operator interface of the reference (src/flash_spacetime/
forward.py): `flash_spacetime_attention`, `flash_spacetime_attention_varlen`,
the test-visible launcher `flash_spacetime_forward` and the autograd
Function, with the same argument meaning, return values, padding contract
(padding rows exactly zero) and errors. The work runs in the gfx950 HIP
library through its C ABI; the projection of the pair embedding (`u = qt W`
before the kernel, `o2 = A' W^T + b` after it, forward.py:279-346) is fused
into the kernel. There is no other backend: a missing library or a CPU
tensor raises.
"""

from __future__ import annotations

import contextlib
import copy
import os
import threading
import weakref
from typing import Any, List, Optional, Tuple

import torch
from torch import Tensor

from . import _lib, tune

_DTYPES = {torch.bfloat16: _lib.FST_BF16, torch.float32: _lib.FST_F32}


def _next_pow2(n: int, floor: int = 16) -> int:
    """Power-of-two bucket (reference _tiles.py:300-304); kept for API parity."""
    p = floor
    while p < n:
        p *= 2
    return p


def lengths_from_mask(mask: Tensor, length: int) -> Tensor:
    """`[B]` int32 valid lengths from a front-packed `[B, L]` padding mask.

    Accepts a bool mask (True marks PADDING, torch.nn.MultiheadAttention's
    `key_padding_mask` convention) or the float mask of the reference's
    `float_padding_mask` (0 valid, -inf padding). The kernels address valid
    tokens as a prefix of each event (forward.py:241-242), so a mask whose
    valid tokens are not a prefix raises ValueError; the check reads one
    flag back from the device.
    """
    if mask.dim() != 2 or mask.shape[1] != length:
        raise ValueError(f"key_padding_mask must be [B, L={length}], got {tuple(mask.shape)}")
    valid = ~mask if mask.dtype == torch.bool else (mask == 0)
    seqlens = valid.sum(1, dtype=torch.int32)
    prefix = torch.arange(length, device=mask.device)[None, :] < seqlens[:, None]
    if not bool(torch.equal(prefix, valid)):
        raise ValueError("key_padding_mask must be front-packed (valid tokens first in every event)")
    return seqlens


def _valid_from_mask(mask: Tensor, length: int) -> Tensor:
    """`[B, L]` bool validity (True = valid token) of a padding mask."""
    if mask.dim() != 2 or mask.shape[1] != length:
        raise ValueError(f"key_padding_mask must be [B, L={length}], got {tuple(mask.shape)}")
    return ~mask if mask.dtype == torch.bool else (mask == 0)


def _is_front_packed(valid: Tensor) -> bool:
    """Whether every event's valid tokens form a prefix (one device readback)."""
    seqlens = valid.sum(1, dtype=torch.int32)
    prefix = torch.arange(valid.shape[1], device=valid.device)[None, :] < seqlens[:, None]
    return bool(torch.equal(prefix, valid))


def is_token_major(t: Tensor) -> bool:
    """Whether a `[B, H, L, D]` tensor is the heads-first view of dense
    `[B, L, H, D]` memory, as `split_heads` leaves a `[B, L, H*D]`
    projection (reference.py:187-191). Such tensors are read in place; a
    tensor that is also contiguous `[B, H, L, D]` (H == 1 or L == 1) counts
    as heads-first."""
    return t.dim() == 4 and not t.is_contiguous() and t.transpose(1, 2).is_contiguous()


def _vec_in_layout(x: Tensor, token_major: bool) -> Tensor:
    """A float32 `[B, H, L]` per-row vector (lse) stored as the kernels read it:
    `[B, L, H]` memory when the operands are token-major."""
    x = x.to(torch.float32)
    if token_major:
        return x if x.transpose(1, 2).is_contiguous() else x.transpose(1, 2).contiguous().transpose(1, 2)
    return x.contiguous()


def _resolve_lengths(seqlens: Optional[Tensor], key_padding_mask: Optional[Tensor], batch: int,
                     length: int) -> Tensor:
    if key_padding_mask is not None and seqlens is not None:
        raise ValueError("pass either seqlens or key_padding_mask, not both")
    if key_padding_mask is not None:
        return lengths_from_mask(key_padding_mask, length)
    if seqlens is None:
        raise ValueError("seqlens (or key_padding_mask) is required")
    if seqlens.dim() == 2:
        return lengths_from_mask(seqlens, length)
    if seqlens.dim() != 1 or seqlens.shape[0] != batch:
        raise ValueError(f"seqlens must be [B={batch}], got {tuple(seqlens.shape)}")
    if seqlens.dtype.is_floating_point or seqlens.dtype == torch.bool:
        raise ValueError(f"seqlens must be an integer tensor, got {seqlens.dtype}")
    return seqlens


_HALF = torch.float16


def _bf16(*ts: Tensor) -> Tuple[Tensor, ...]:
    """float16 operands for the bf16 kernels. The reference computes every
    operand that is not float32 in bf16 (forward.py:271, backward.py:523:
    `compute_bf16 = q.dtype != torch.float32`), so float16 inputs run the
    bf16 path and results go back to float16. `to` keeps a dense view's
    strides, so token-major views stay token-major."""
    return tuple(t.to(torch.bfloat16) for t in ts)


def head_groups(dtype: int, heads: int, dim: int, channels: int) -> List[Tuple[int, int]]:
    """Head ranges [h0, h1) the kernels run one call each: all heads at once
    where the library has a kernel for that many, else the fewest equal
    groups (sizes differing by at most one) it has one for -- more than 16
    heads, or float32 at D = C = 64 with more than 8. The reference pads heads
    to the next power of two inside one kernel and takes any count
    (forward.py:22, backward.py:574)."""
    lib = _lib.load()
    for n in range(1, heads + 1):
        if lib.fst_supported(dtype, -(-heads // n), dim, channels):
            bounds = [i * heads // n for i in range(n + 1)]
            return [(bounds[i], bounds[i + 1]) for i in range(n)]
    raise ValueError(f"no kernel for head_dim {dim} and C={channels} in this dtype")


class _Prepared:
    """Validated kernel operands shared by forward and backward.

    Padded q, k, v that are all heads-first views of `[B, L, H, D]` memory
    (`is_token_major`) are used in place and the library is told so
    (FST_TOKEN_MAJOR); the outputs, gradients and lse then come back as the
    same kind of view. Anything else is made contiguous `[B, H, L, D]`, as
    the reference does (forward.py:274)."""

    def __init__(self, q, k, v, feats, weight, bias, seqlens, scale, use_attn_bias,
                 use_activation_bias, cu_seqlens, interleaved: bool = False):
        for t in (q, k, v, feats, weight):
            _lib.require_gpu(t)
        if q.dtype not in _DTYPES:
            raise ValueError(f"q must be bfloat16 or float32, got {q.dtype}")
        if k.dtype != q.dtype or v.dtype != q.dtype:
            raise ValueError("q, k and v must share one dtype")
        self.packed = cu_seqlens is not None
        if self.packed:
            if q.dim() != 3:
                raise ValueError(f"packed q must be [T, H, D], got {tuple(q.shape)}")
            total, heads, dim = q.shape
            self.batch = int(cu_seqlens.numel()) - 1
            self.length = 0
            self.tokens = total
            lens = cu_seqlens
            if feats.dim() != 2 or feats.shape[0] != total:
                raise ValueError(f"packed feats must be [T={total}, F>=4], got {tuple(feats.shape)}")
        else:
            if q.dim() != 4:
                raise ValueError(f"q must be [B, H, L, D], got {tuple(q.shape)}")
            self.batch, heads, self.length, dim = q.shape
            self.tokens = 0
            lens = _resolve_lengths(seqlens, None, self.batch, self.length)
            if feats.dim() != 3 or feats.shape[:2] != (self.batch, self.length):
                raise ValueError(f"feats must be [B, L, F>=4], got {tuple(feats.shape)}")
        if k.shape != q.shape or v.shape != q.shape:
            raise ValueError("q, k and v must have the same shape")
        if feats.shape[-1] < 4:
            raise ValueError("feats needs at least 4 columns (x, y, z, t)")
        if weight.dim() != 2 or weight.shape[0] != dim:
            raise ValueError(f"weight must be [D={dim}, C] (nn.Linear layout), got {tuple(weight.shape)}")
        c = weight.shape[1]
        if c not in (16, 32, 48, 64):
            raise ValueError(f"kernel supports C in (16, 32, 48, 64), got {c}")
        if dim not in (16, 32, 48, 64):
            raise ValueError(f"kernel supports head_dim in (16, 32, 48, 64), got {dim}")
        if heads < 1:
            raise ValueError(f"need at least one head, got {heads}")
        if bias is not None and bias.shape != (dim,):
            raise ValueError(f"bias must be [D={dim}], got {tuple(bias.shape)}")
        self.heads, self.dim, self.channels = heads, dim, c
        self.dtype = _DTYPES[q.dtype]
        self.groups = head_groups(self.dtype, heads, dim, c)
        self.scale = float(dim ** -0.5 if scale is None else scale)
        # interleaved: q, k, v are the slots of one [B, L, 3, H, D] / [T, 3, H, D]
        # tensor (the caller, `_FlashSpacetimeAttentionQKV`, guarantees it).
        self.interleaved = interleaved
        self.token_major = not self.packed and (interleaved or all(is_token_major(t) for t in (q, k, v)))
        self.flags = ((_lib.FST_ATTN_BIAS if use_attn_bias else 0)
                      | (_lib.FST_ACT_BIAS if use_activation_bias else 0)
                      | (_lib.FST_PACKED if self.packed else 0)
                      | (_lib.FST_TOKEN_MAJOR if self.token_major else 0)
                      | (_lib.FST_QKV_INTERLEAVED if interleaved else 0))
        if self.token_major or interleaved:
            self.q, self.k, self.v = q, k, v
        else:
            self.q, self.k, self.v = (t.contiguous() for t in (q, k, v))
        self.pos4 = feats[..., :4].to(torch.float32).contiguous()
        self.weight = weight.detach().to(torch.float32).contiguous()
        self.bias = bias.detach().to(torch.float32).contiguous() if bias is not None else None
        self.lens = lens.to(device=q.device, dtype=torch.int32).contiguous()
        self.device = q.device
        # The kernels address one event's rows (all heads; q, k, v and the
        # C-wide scratch) with 32-bit byte offsets. The C library refuses
        # padded events past that, and for packed events writes NaN into the
        # rows of an event past it; packed lengths live on the device, so the
        # longest event is read back (to raise instead) only when the whole
        # batch could reach the limit.
        row_bytes = heads * q.element_size() * max(dim * (3 if interleaved else 1), c)
        if self.packed and self.tokens * row_bytes >= 2 ** 31:
            longest = int((self.lens[1:] - self.lens[:-1]).max()) if self.batch > 0 else 0
            if longest * row_bytes >= 2 ** 31:
                raise ValueError(f"an event of {longest} tokens spans {longest * row_bytes} bytes; the kernels "
                                 f"address at most 2^31 - 1 per event")

    def dims(self):
        return (self.dtype, self.flags, self.batch, self.heads, self.length, self.tokens,
                self.dim, self.channels)

    def vec_shape(self):
        if self.packed:
            return (self.tokens, self.heads)
        return (self.batch, self.heads, self.length)

    def empty_out(self) -> Tensor:
        """The output (and grad_out) in the layout the kernels write: q's, or
        for interleaved operands the dense token-major one."""
        if not self.interleaved:
            return torch.empty_like(self.q)
        if self.packed:
            return torch.empty(self.tokens, self.heads, self.dim, device=self.device, dtype=self.q.dtype)
        return torch.empty(self.batch, self.length, self.heads, self.dim, device=self.device,
                           dtype=self.q.dtype).transpose(1, 2)

    def head_slice(self, h0: int, h1: int) -> "_Prepared":
        """The operands of heads [h0, h1) as contiguous tensors of their own
        (heads-first padded or packed, no longer token-major or interleaved)."""
        sub = copy.copy(self)
        sub.q, sub.k, sub.v = (t[:, h0:h1].contiguous() for t in (self.q, self.k, self.v))
        sub.heads = h1 - h0
        sub.token_major = sub.interleaved = False
        sub.flags = self.flags & ~(_lib.FST_TOKEN_MAJOR | _lib.FST_QKV_INTERLEAVED)
        sub.groups = [(0, h1 - h0)]
        return sub

    def empty_vec(self) -> Tensor:
        """A float32 per-row vector (lse, rowsum) in the operands' layout."""
        if self.token_major:
            b, h, length = self.vec_shape()
            return torch.empty(b, length, h, device=self.device, dtype=torch.float32).transpose(1, 2)
        return torch.empty(self.vec_shape(), device=self.device, dtype=torch.float32)


def _run_forward(prep: _Prepared) -> Tuple[Tensor, Tensor]:
    lib = _lib.load()
    out = prep.empty_out()
    lse = prep.empty_vec()
    if len(prep.groups) > 1:
        for h0, h1 in prep.groups:
            o, l_ = _run_forward(prep.head_slice(h0, h1))
            out[:, h0:h1].copy_(o)
            lse[:, h0:h1].copy_(l_)
        return out, lse
    dims = prep.dims()
    ws_bytes = lib.fst_forward_workspace_bytes(*dims)
    ws = torch.empty(max(ws_bytes, 1), device=prep.device, dtype=torch.uint8)

    def run(flags: int) -> int:
        return lib.fst_forward(
            dims[0], flags, *dims[2:],
            _lib.ptr(prep.q), _lib.ptr(prep.k), _lib.ptr(prep.v), _lib.ptr(prep.pos4),
            _lib.ptr(prep.weight), _lib.ptr(prep.bias), _lib.ptr(prep.lens), prep.scale,
            _lib.ptr(out), _lib.ptr(lse), _lib.ptr(ws), ws_bytes, _lib.stream_handle(prep.device),
        )

    with torch.cuda.device(prep.device):
        plan = tune.forward_plan(dims, run)
        rc = run(dims[1] | plan)
    _lib.check(rc, "flash_spacetime_forward")
    return out, lse


def flash_spacetime_forward(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    feats: Tensor,
    weight: Tensor,
    bias: Optional[Tensor],
    seqlens: Optional[Tensor],
    scale: Optional[float] = None,
    use_attn_bias: bool = True,
    use_activation_bias: bool = True,
    block_m: Optional[int] = None,
    block_n: Optional[int] = None,
    num_warps: Optional[int] = None,
    num_stages: Optional[int] = None,
    cu_seqlens: Optional[Tensor] = None,
) -> Tuple[Tensor, Tensor]:
    """Fused forward: (out `[B, H, L, D]` with padding rows 0, lse `[B, H, L]`).

    Same contract as the reference launcher (forward.py:222-346): `seqlens`
    is the `[B]` integer tensor of valid lengths (a front-packed `[B, L]`
    padding mask is also accepted); with `cu_seqlens` (`[B+1]` token
    offsets) the tensors are packed `[T, H, D]` / `[T, F]` and `seqlens` is
    ignored. `weight` is `[D, C]` (nn.Linear layout; the reference's
    `[C, C]` with C == D is the special case). lse excludes the row-constant
    `qt . b` term, as the reference kernel's does. The reference's tile
    arguments select compiled kernel variants (tune.plan_from_tiles): block_m
    the float32 kernel's query rows per workgroup, block_n its keys per chunk
    (16 or 32; the bf16 kernel's too), each the nearest offered value. None
    (the default here; the reference defaults to 16 / 32 bf16, 16 fp32)
    keeps the library's tuned or static choice. num_warps has no forward
    counterpart (the kernels run four waves per workgroup) and num_stages
    none at all (loads run one chunk ahead); both are accepted.
    """
    del num_stages
    if q.dtype == _HALF:
        out, lse = flash_spacetime_forward(*_bf16(q, k, v), feats, weight, bias, seqlens, scale, use_attn_bias,
                                           use_activation_bias, block_m=block_m, block_n=block_n,
                                           num_warps=num_warps, cu_seqlens=cu_seqlens)
        return out.to(_HALF), lse
    prep = _Prepared(q, k, v, feats, weight, bias, seqlens, scale, use_attn_bias,
                     use_activation_bias, cu_seqlens)
    with tune.tile_request(block_m, block_n, None):
        return _run_forward(prep)


_TEMPORARY_OUTPUT = threading.local()


@contextlib.contextmanager
def _output_is_temporary():
    """Calls inside convert or scatter the op's output into another tensor
    (float16 results, masks with holes): their backward keeps nothing of the
    output, and the rows kernel forms D online."""
    prev = getattr(_TEMPORARY_OUTPUT, "on", False)
    _TEMPORARY_OUTPUT.on = True
    try:
        yield
    finally:
        _TEMPORARY_OUTPUT.on = prev


def _keep_output(ctx: Any, out: Tensor, returned: Optional[Tensor] = None) -> List[Tensor]:
    """What of the forward's output the backward keeps, to be appended to the
    tensors saved for backward: the bf16 rows kernel takes its reference D
    from it. It goes through save_for_backward (so saved-tensor hooks, such as
    offloading or checkpointing, handle it like any saved tensor) as `.data`,
    an alias with a version counter of its own, so that modifying the output
    in place does not make the backward fail as it would for a saved output.
    A weak reference to the tensor the caller receives (`returned`, default
    `out`) and its version tell the backward whether the caller modified it
    since; nothing is kept where the output is a temporary of the op."""
    if getattr(_TEMPORARY_OUTPUT, "on", False):
        ctx.out_ref = None
        return []
    ret = out if returned is None else returned
    ctx.out_ref = weakref.ref(ret)
    ctx.out_version = ret._version
    return [out.data]


def _kept_output(ctx: Any, kept: Tuple[Tensor, ...]) -> Optional[Tensor]:
    """The kept output (the saved tensors past the inputs and lse), or None
    where nothing was kept or the caller modified the output in place since
    the forward; then the kernel forms D online. Either way D is the kernel's
    own N / Z, so the gradients do not depend on which (a caller that
    modified the output and then dropped it leaves the modified values as the
    reference, which moves only roundings)."""
    if not kept:
        return None
    ret = None if ctx.out_ref is None else ctx.out_ref()
    if ret is not None and ret._version != ctx.out_version:
        return None
    return kept[0]


class _FlashSpacetimeAttention(torch.autograd.Function):
    """Fused forward and deterministic HIP backward (forward.py:349-478)."""

    @staticmethod
    def forward(  # type: ignore[override]
        ctx: Any,
        q: Tensor,
        k: Tensor,
        v: Tensor,
        feats: Tensor,
        weight: Tensor,
        bias: Optional[Tensor],
        seqlens: Optional[Tensor],
        scale: Optional[float],
        use_attn_bias: bool,
        use_activation_bias: bool,
        cu_seqlens: Optional[Tensor] = None,
    ) -> Tensor:
        if feats.requires_grad:
            raise ValueError("feats (detector data) must not require grad")
        prep = _Prepared(q, k, v, feats, weight, bias, seqlens, scale, use_attn_bias,
                         use_activation_bias, cu_seqlens)
        out, lse = _run_forward(prep)
        # The inputs and the LSE are saved as the reference saves them
        # (forward.py:381-388); the backward forms its own softmax row sums.
        ctx.save_for_backward(prep.q, prep.k, prep.v, prep.pos4, prep.lens, lse, *_keep_output(ctx, out))
        ctx.prep_meta = (prep.weight, prep.bias, weight.dtype,
                         None if bias is None else bias.dtype)
        ctx.dims = prep.dims()
        ctx.scale = prep.scale
        ctx.packed = prep.packed
        ctx.flags = (use_attn_bias, use_activation_bias)
        ctx.vec_shape = prep.vec_shape()
        return out

    @staticmethod
    def backward(ctx: Any, grad_out: Tensor) -> Tuple[Optional[Tensor], ...]:  # type: ignore[override]
        if os.environ.get("FLASH_ST_REFERENCE_BWD", "0") == "1":
            raise RuntimeError(
                "FLASH_ST_REFERENCE_BWD=1 (autograd through the materialised reference) is not "
                "offered: this build has only the fused HIP backward"
            )
        from .backward import _run_backward

        q, k, v, pos4, lens, lse, *kept = ctx.saved_tensors
        w32, b32, w_dtype, b_dtype = ctx.prep_meta
        dq, dk, dv, dw, db = _run_backward(
            ctx.dims, q, k, v, pos4, w32, b32, lens, lse, grad_out, ctx.scale, ctx.vec_shape,
            out=_kept_output(ctx, kept),
        )
        use_attn_bias, use_activation_bias = ctx.flags
        proj_used = use_attn_bias or use_activation_bias
        w_needed, b_needed = ctx.needs_input_grad[4], ctx.needs_input_grad[5]
        return (
            dq if ctx.needs_input_grad[0] else None,
            dk if ctx.needs_input_grad[1] else None,
            dv if ctx.needs_input_grad[2] else None,
            None,
            dw.to(w_dtype) if (w_needed and proj_used) else None,
            db.to(b_dtype) if (b_needed and proj_used and db is not None) else None,
            None, None, None, None, None,
        )


def flash_spacetime_attention(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    feats: Tensor,
    weight: Tensor,
    bias: Optional[Tensor],
    seqlens: Optional[Tensor] = None,
    scale: Optional[float] = None,
    use_attn_bias: bool = True,
    use_activation_bias: bool = True,
    *,
    key_padding_mask: Optional[Tensor] = None,
) -> Tensor:
    """Fused spacetime-bias attention (public op, forward.py:481-501).

    Semantics of `spacetime_attention_reference` on valid rows; padding rows
    of the output are exactly zero. The 7th argument is the `[B]` integer
    tensor of valid lengths; a `[B, L]` padding mask (bool, True = padding,
    or the 0 / -inf float mask) may be given instead, positionally or as
    `key_padding_mask=`. A front-packed mask becomes lengths (one readback);
    a mask with holes runs the packed kernels on the gathered valid tokens.
    """
    if q.dtype == _HALF:
        with _output_is_temporary():
            out = flash_spacetime_attention(*_bf16(q, k, v), feats, weight, bias, seqlens, scale, use_attn_bias,
                                            use_activation_bias, key_padding_mask=key_padding_mask)
        return out.to(_HALF)
    mask = key_padding_mask
    if mask is None and seqlens is not None and seqlens.dim() == 2:
        mask = seqlens
        seqlens = None
    if mask is not None:
        if seqlens is not None:
            raise ValueError("pass either seqlens or key_padding_mask, not both")
        valid = _valid_from_mask(mask, q.shape[2])
        if not _is_front_packed(valid):
            return _attention_scattered(q, k, v, feats, weight, bias, valid, scale, use_attn_bias,
                                        use_activation_bias)
        seqlens = valid.sum(1, dtype=torch.int32)
    return _FlashSpacetimeAttention.apply(
        q, k, v, feats, weight, bias, seqlens, scale, use_attn_bias, use_activation_bias, None
    )


def _attention_scattered(q, k, v, feats, weight, bias, valid, scale, use_attn_bias, use_activation_bias):
    """A padding mask whose valid tokens are not a prefix of each event.

    The spec's semantics (reference.py:106-167: padding keys masked out,
    padding rows zero in the kernel's contract) depend only on which tokens
    are valid and on their features, not on their slots: the valid tokens of
    every event are gathered in order into the packed layout, run through the
    packed kernels, and the rows scattered back (padding rows zero). The
    gather and scatter are torch index operations on the device and reading
    the token count back is one host synchronisation.
    """
    b, h, length, d = q.shape
    if feats.dim() != 3 or feats.shape[:2] != (b, length):
        raise ValueError(f"feats must be [B, L, F>=4], got {tuple(feats.shape)}")
    counts = valid.sum(1, dtype=torch.int32)
    cu = torch.zeros(b + 1, dtype=torch.int32, device=q.device)
    cu[1:] = torch.cumsum(counts, 0, dtype=torch.int32)
    rows = lambda x: x.transpose(1, 2)[valid]  # [T, H, D], events and tokens in order
    with _output_is_temporary():  # scattered into the padded result below
        out = flash_spacetime_attention_varlen(rows(q), rows(k), rows(v), feats[valid], weight, bias, cu, scale,
                                               use_attn_bias, use_activation_bias)
    full = out.new_zeros(b, length, h, d).index_put((valid,), out)
    # Heads-first view of the token-major result when q was one, else
    # contiguous [B, H, L, D].
    return full.transpose(1, 2) if is_token_major(q) else full.transpose(1, 2).contiguous()


def flash_spacetime_attention_varlen(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    feats: Tensor,
    weight: Tensor,
    bias: Optional[Tensor],
    cu_seqlens: Optional[Tensor] = None,
    scale: Optional[float] = None,
    use_attn_bias: bool = True,
    use_activation_bias: bool = True,
) -> Tensor:
    """Packed (uncapped) fused spacetime-bias attention (forward.py:504-527).

    q/k/v are `[T, H, D]` and feats `[T, F]` with events delimited by
    `cu_seqlens` (`[B+1]` token offsets, cu[0] = 0, cu[-1] = T) -- the values
    layout of a jagged NestedTensor. No padding exists and event lengths are
    unbounded; nothing is read back to the host.

    q, k and v may instead be `torch.nested` jagged tensors `[B, j, H, D]`
    (feats jagged `[B, j, F]` or its `[T, F]` values): the events are then
    the nested tensor's, `cu_seqlens` may be omitted (or must equal its
    offsets), and the output is a jagged tensor with the same offsets.
    """
    if q.dtype == _HALF:
        with _output_is_temporary():
            out = flash_spacetime_attention_varlen(*_bf16(q, k, v), feats, weight, bias, cu_seqlens, scale,
                                                   use_attn_bias, use_activation_bias)
        return out.to(_HALF)
    if q.is_nested:
        if not (k.is_nested and v.is_nested):
            raise ValueError("q, k and v must all be nested tensors, or none of them")
        if q.layout != torch.jagged or q.dim() != 4:
            raise ValueError("nested q, k, v must be jagged [B, j, H, D] tensors (torch.jagged layout)")
        offsets = q.offsets()
        if cu_seqlens is None:
            cu_seqlens = offsets
        fv = feats.values() if feats.is_nested else feats
        out = _FlashSpacetimeAttention.apply(
            q.values(), k.values(), v.values(), fv, weight, bias, None, scale, use_attn_bias,
            use_activation_bias, cu_seqlens
        )
        return torch.nested.nested_tensor_from_jagged(out, offsets)
    if cu_seqlens is None:
        raise ValueError("cu_seqlens is required for dense packed inputs")
    return _FlashSpacetimeAttention.apply(
        q, k, v, feats, weight, bias, None, scale, use_attn_bias, use_activation_bias, cu_seqlens
    )


def _qkv_views(qkv: Tensor, packed: bool) -> Tuple[Tensor, Tensor, Tensor]:
    """q, k, v as the kernels index them: `[T, H, D]` slots of a packed
    `[T, 3, H, D]`, or heads-first `[B, H, L, D]` views of `[B, L, 3, H, D]`."""
    if packed:
        return qkv[:, 0], qkv[:, 1], qkv[:, 2]
    return qkv[:, :, 0].transpose(1, 2), qkv[:, :, 1].transpose(1, 2), qkv[:, :, 2].transpose(1, 2)


class _FlashSpacetimeAttentionQKV(torch.autograd.Function):
    """The fused op on one interleaved q/k/v tensor; its gradient is one
    tensor of the same layout, written by the kernels slot by slot."""

    @staticmethod
    def forward(  # type: ignore[override]
        ctx: Any,
        qkv: Tensor,
        feats: Tensor,
        weight: Tensor,
        bias: Optional[Tensor],
        seqlens: Optional[Tensor],
        scale: Optional[float],
        use_attn_bias: bool,
        use_activation_bias: bool,
        cu_seqlens: Optional[Tensor],
    ) -> Tensor:
        if feats.requires_grad:
            raise ValueError("feats (detector data) must not require grad")
        packed = cu_seqlens is not None
        q, k, v = _qkv_views(qkv, packed)
        prep = _Prepared(q, k, v, feats, weight, bias, seqlens, scale, use_attn_bias,
                         use_activation_bias, cu_seqlens, interleaved=True)
        out, lse = _run_forward(prep)
        ret = out if packed else out.transpose(1, 2)  # [T, H, D] / [B, L, H, D], dense
        ctx.save_for_backward(qkv, prep.pos4, prep.lens, lse, *_keep_output(ctx, out, ret))
        ctx.prep_meta = (prep.weight, prep.bias, weight.dtype, None if bias is None else bias.dtype)
        ctx.dims = prep.dims()
        ctx.scale = prep.scale
        ctx.packed = packed
        ctx.flags = (use_attn_bias, use_activation_bias)
        ctx.vec_shape = prep.vec_shape()
        return ret

    @staticmethod
    def backward(ctx: Any, grad_out: Tensor) -> Tuple[Optional[Tensor], ...]:  # type: ignore[override]
        from .backward import _run_backward

        qkv, pos4, lens, lse, *kept = ctx.saved_tensors
        w32, b32, w_dtype, b_dtype = ctx.prep_meta
        q, k, v = _qkv_views(qkv, ctx.packed)
        dqkv = torch.empty_like(qkv)
        g = grad_out if ctx.packed else grad_out.transpose(1, 2)
        if ctx.packed:
            like = torch.empty(q.shape, device=qkv.device, dtype=qkv.dtype)
        else:
            b, h, length, d = q.shape
            like = torch.empty(b, length, h, d, device=qkv.device, dtype=qkv.dtype).transpose(1, 2)
        _, _, _, dw, db = _run_backward(
            ctx.dims, q, k, v, pos4, w32, b32, lens, lse, g, ctx.scale, ctx.vec_shape,
            out_like=like, grads=_qkv_views(dqkv, ctx.packed), out=_kept_output(ctx, kept),
        )
        use_attn_bias, use_activation_bias = ctx.flags
        proj_used = use_attn_bias or use_activation_bias
        return (
            dqkv if ctx.needs_input_grad[0] else None,
            None,
            dw.to(w_dtype) if (ctx.needs_input_grad[2] and proj_used) else None,
            db.to(b_dtype) if (ctx.needs_input_grad[3] and proj_used and db is not None) else None,
            None, None, None, None, None,
        )


def flash_spacetime_attention_qkv(
    qkv: Tensor,
    feats: Tensor,
    weight: Tensor,
    bias: Optional[Tensor],
    seqlens: Optional[Tensor] = None,
    scale: Optional[float] = None,
    use_attn_bias: bool = True,
    use_activation_bias: bool = True,
    *,
    cu_seqlens: Optional[Tensor] = None,
    key_padding_mask: Optional[Tensor] = None,
) -> Tensor:
    """The fused op on the output of one fused q/k/v projection.

    `qkv` is `[B, L, 3, H, D]` (padded; a `[B, L, 3*H*D]` linear's output
    viewed so) or `[T, 3, H, D]` with `cu_seqlens` (packed). The kernels read
    the three slots in place and write the gradient as one tensor of the same
    layout, so neither the projection's output nor its gradient is copied,
    split or stacked. Returns `[B, L, H, D]` (padding rows zero) or
    `[T, H, D]`: the layout the output projection consumes. Lengths and
    masks as in `flash_spacetime_attention` (a mask with holes runs the
    packed path on the gathered valid tokens). Same values as
    `flash_spacetime_attention(q, k, v, ...)` on the split heads. No
    reference counterpart: the reference takes three separate tensors
    (forward.py:481-501).
    """
    if qkv.dtype == _HALF:
        with _output_is_temporary():
            out = flash_spacetime_attention_qkv(qkv.to(torch.bfloat16), feats, weight, bias, seqlens, scale,
                                                use_attn_bias, use_activation_bias, cu_seqlens=cu_seqlens,
                                                key_padding_mask=key_padding_mask)
        return out.to(_HALF)
    if cu_seqlens is not None:
        if qkv.dim() != 4 or qkv.shape[1] != 3:
            raise ValueError(f"packed qkv must be [T, 3, H, D], got {tuple(qkv.shape)}")
        return _FlashSpacetimeAttentionQKV.apply(
            qkv.contiguous(), feats, weight, bias, None, scale, use_attn_bias, use_activation_bias,
            cu_seqlens,
        )
    if qkv.dim() != 5 or qkv.shape[2] != 3:
        raise ValueError(f"qkv must be [B, L, 3, H, D], got {tuple(qkv.shape)}")
    mask = key_padding_mask
    if mask is None and seqlens is not None and seqlens.dim() == 2:
        mask, seqlens = seqlens, None
    if mask is not None:
        if seqlens is not None:
            raise ValueError("pass either seqlens or key_padding_mask, not both")
        b, length = qkv.shape[:2]
        valid = _valid_from_mask(mask, length)
        if not _is_front_packed(valid):
            if feats.dim() != 3 or feats.shape[:2] != (b, length):
                raise ValueError(f"feats must be [B, L, F>=4], got {tuple(feats.shape)}")
            cu = torch.zeros(b + 1, dtype=torch.int32, device=qkv.device)
            cu[1:] = torch.cumsum(valid.sum(1, dtype=torch.int32), 0, dtype=torch.int32)
            with _output_is_temporary():  # scattered into the padded result below
                out = _FlashSpacetimeAttentionQKV.apply(
                    qkv[valid], feats[valid], weight, bias, None, scale, use_attn_bias,
                    use_activation_bias, cu,
                )
            return out.new_zeros(b, length, *out.shape[1:]).index_put((valid,), out)
        seqlens = valid.sum(1, dtype=torch.int32)
    return _FlashSpacetimeAttentionQKV.apply(
        qkv.contiguous(), feats, weight, bias, seqlens, scale, use_attn_bias, use_activation_bias, None,
    )
