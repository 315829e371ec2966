"""CPU restatement of the flash-spacetime specification (test infrastructure).

Every function cites the reference line it restates; paths are relative to
the sevmag/flash-spacetime checkout. The reference requires `W [C, C]` with
`C == D` (reference.py:139-143); this restatement takes the nn.Linear layout
`W [D, C]` so the BASELINE configurations (D=32, C=16; D=C=64) are
expressible. With `C == D` it reduces to the reference exactly, which the
golden-vector tests check.

Two evaluators live here:

* `attention` -- the eager definition with the reference's dtype plumbing
  (emb -> weight dtype, fp32-mask promotion, `p.to(v.dtype)`), used at small
  shapes and in any dtype, and as the CPU baseline's workload.
* `attention_fp64_chunked` / `backward_fp64_chunked` -- float64, per event
  and per block of query rows, valid tokens only, so configurations whose
  `[B, L, L, D]` pair tensor would need tens of GiB stay within a few
  hundred MiB. The backward is the closed-form gradient of the spec,
  written out term by term (checked against autograd in the tests).
"""

from __future__ import annotations

import math
from typing import Optional, Sequence, Tuple

import torch
from torch import Tensor

# reference.py:39-42. 3e4 / 500 * 3e-1 evaluates to exactly 18.0 in binary64
# and the value survives the fp32 cast unchanged.
TIME_SCALE = 3e4 / 500 * 3e-1
SINEMB_INPUT_SCALE = 1024.0
SINEMB_CLIP = 4.0
SINEMB_N_FREQ = 10000.0


def frequencies(c: int) -> Tensor:
    """fp32 frequency ladder `exp(-i * ln(1e4) / (c/2))`, i < c/2.

    reference.py:45-56 forms the ladder in float32 whatever the working dtype:
    fp32 log of 1e4, divided by the float c/2, times an fp32 arange,
    exponentiated in fp32. The same fp32 steps are taken here, with the two
    transcendental steps correctly rounded (evaluated in binary64, rounded
    once to fp32). torch's vectorised fp32 exp is not correctly rounded and
    differs between CPUs by an ulp on some entries (seen: C=64 i=11 in one
    container, i=3 on another host); a correctly rounded ladder makes the
    oracle machine-independent and equal to the GPU library's ladder. The
    golden-vector test pins it bitwise to the reference wherever the
    reference's own evaluation was correctly rounded, and to within one ulp
    elsewhere.
    """
    if c <= 0 or c % 2:
        raise ValueError(f"channel count must be positive and even, got {c}")
    half = c / 2
    log_n = torch.tensor([math.log(SINEMB_N_FREQ)], dtype=torch.float64).float()
    neg_log_step = -(log_n / half)
    ramp = torch.arange(half, dtype=torch.float32)
    return torch.exp((ramp * neg_log_step).double()).float()


def pair_angle_rect(rows: Tensor, cols: Tensor) -> Tensor:
    """`x_ij = 1024 * clip(sign(I) sqrt|I|, -4, 4)`, `[B, M, N]` from `[B, M, F]`, `[B, N, F]`.

    reference.py:75-81 with `I = |p_i - p_j|^2 - (18 (t_i - t_j))^2`;
    positions are columns 0-2 and the interval's time is column 3. The
    computation runs in the dtype of the features.
    """
    spatial = (rows[:, :, None, :3] - cols[:, None, :, :3]).pow(2).sum(-1)
    temporal = ((rows[:, :, None, 3] - cols[:, None, :, 3]) * TIME_SCALE).pow(2)
    interval = spatial - temporal
    signed = torch.sign(interval) * torch.sqrt(torch.abs(interval))
    return SINEMB_INPUT_SCALE * signed.clip(-SINEMB_CLIP, SINEMB_CLIP)


def pair_angle(feats: Tensor) -> Tensor:
    """All-pairs angle `[B, L, L]` of `[B, L, F]` feats (reference.py:75-81)."""
    return pair_angle_rect(feats, feats)


def embed_angle(x: Tensor, c: int) -> Tensor:
    """`[sin(x f), cos(x f)]` along a new last axis of width C (reference.py:82-84)."""
    theta = x.unsqueeze(-1) * frequencies(c).to(x.device)
    return torch.cat((torch.sin(theta), torch.cos(theta)), dim=-1)


def pair_embedding(feats: Tensor, c: int) -> Tensor:
    """`E_ij = [sin(x f), cos(x f)]`, `[B, L, L, C]` in the feats dtype.

    reference.py:82-84: the fp32 ladder multiplies the angle (promoting to
    float64 when feats are float64); sin channels first, then cos.
    """
    return embed_angle(pair_angle(feats), c)


def pair_features(feats: Tensor, weight: Tensor, bias: Optional[Tensor]) -> Tensor:
    """`R_ij = W E_ij + b`, `[B, L, L, D]` for `W [D, C]` (nn.Linear layout).

    reference.py:59-88: the embedding is cast to the weight dtype before the
    projection, which runs in that dtype.
    """
    emb = pair_embedding(feats, weight.shape[1])
    return torch.nn.functional.linear(emb.to(weight.dtype), weight, bias)


def pair_mask(key_padding_mask: Tensor) -> Tensor:
    """`[B, L, L]` additive mask: -inf where exactly one token is padding.

    reference.py:91-103. Pairs of two padding tokens stay 0 (their rows are
    padding rows, which the fused op zeroes and the tests never compare).
    """
    row = key_padding_mask[:, :, None]
    col = key_padding_mask[:, None, :]
    out = torch.minimum(row, col).clone()
    out[torch.maximum(row, col) < 0] = 0
    return out


def valid_row_mask(batch: int, length: int, seqlens: Tensor) -> Tensor:
    """`[B, L]` booleans, True on the first `seqlens[b]` tokens (reference.py:170-177)."""
    pos = torch.arange(length, device=seqlens.device)
    return pos[None, :] < seqlens[:, None]


def float_padding_mask(valid: Tensor, dtype: torch.dtype) -> Tensor:
    """0 on valid tokens, -inf on padding (reference.py:180-184)."""
    out = torch.zeros(valid.shape, dtype=dtype, device=valid.device)
    out.masked_fill_(~valid, float("-inf"))
    return out


def attention(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    feats: Tensor,
    weight: Tensor,
    bias: Optional[Tensor],
    key_padding_mask: Optional[Tensor] = None,
    scale: Optional[float] = None,
    use_attn_bias: bool = True,
    use_activation_bias: bool = True,
) -> Tensor:
    """Eager spacetime-bias attention (reference.py:106-167, W generalised).

    q, k, v: `[B, H, L, D]`; feats `[B, L, F]`; weight `[D, C]`; bias `[D]`.
    Materialises the `[B, L, L, D]` pair tensor and the `[B, H, L, L]`
    logits, so it is for small shapes and for the CPU baseline only.
    """
    head_dim = q.shape[-1]
    if weight.shape[0] != head_dim:
        raise ValueError(f"weight must be [D={head_dim}, C], got {tuple(weight.shape)}")
    s = head_dim ** -0.5 if scale is None else scale
    qt = q * s
    logits = qt @ k.transpose(-2, -1)
    rel = None
    if use_attn_bias or use_activation_bias:
        rel = pair_features(feats, weight, bias)
    if use_attn_bias:
        logits = logits + torch.einsum("bhid,bijd->bhij", qt, rel)
    if key_padding_mask is not None:
        logits = logits + pair_mask(key_padding_mask).unsqueeze(1)
    probs = logits.softmax(dim=-1)
    out = probs.to(v.dtype) @ v
    if use_activation_bias:
        out = out + torch.einsum("bhij,bijd->bhid", probs.to(rel.dtype), rel)
    return out


# ---------------------------------------------------------------------------
# Chunked float64 evaluation (valid tokens only).
# ---------------------------------------------------------------------------


def _event_slices(
    seqlens: Optional[Tensor], cu_seqlens: Optional[Tensor], batch: int, length: int
) -> Sequence[Tuple[int, int]]:
    """(start, length) of each event: padded rows [0, l) or packed tokens."""
    if cu_seqlens is not None:
        cu = [int(x) for x in cu_seqlens.tolist()]
        return [(cu[i], cu[i + 1] - cu[i]) for i in range(len(cu) - 1)]
    lens = [int(x) for x in seqlens.tolist()] if seqlens is not None else [length] * batch
    return [(0, n) for n in lens]


def _gather_event(x: Tensor, b: int, start: int, n: int, packed: bool) -> Tensor:
    """`[H, n, X]` rows of event b from `[B, H, L, X]` or packed `[T, H, X]`."""
    if packed:
        return x[start:start + n].transpose(0, 1)
    return x[b, :, :n]


def _event_feats(feats: Tensor, b: int, start: int, n: int, packed: bool) -> Tensor:
    return feats[start:start + n] if packed else feats[b, :n]


def _row_block_pair_terms(
    feats_rows: Tensor, feats_all: Tensor, weight64: Tensor, bias64: Optional[Tensor]
) -> Tuple[Tensor, Tensor]:
    """E `[m, n, C]` and R `[m, n, D]` in float64 for a block of query rows."""
    x = pair_angle_rect(feats_rows.double()[None], feats_all.double()[None])[0]
    emb = embed_angle(x, weight64.shape[1])
    rel = emb @ weight64.t()
    if bias64 is not None:
        rel = rel + bias64
    return emb, rel


def attention_fp64_chunked(
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
    cu_seqlens: Optional[Tensor] = None,
    row_block: int = 256,
) -> Tuple[Tensor, Tensor]:
    """float64 forward of the spec on valid rows: (out, lse).

    Layout follows the fused op: padded `[B, H, L, D]` with `seqlens`, or
    packed `[T, H, D]` with `cu_seqlens`. Padding rows of `out` and `lse`
    are 0 (the fused op's contract, forward.py:19-22). The log-sum-exp is
    over the logits that include the `qt.b` term; the fused kernel drops
    that row constant, so its LSE differs by exactly `qt_i . b`.
    """
    packed = cu_seqlens is not None
    head_dim = q.shape[-1]
    s = head_dim ** -0.5 if scale is None else scale
    batch = 0 if packed else q.shape[0]
    length = 0 if packed else q.shape[2]
    out = torch.zeros(q.shape, dtype=torch.float64)
    lse = torch.zeros(q.shape[:-1], dtype=torch.float64)
    w64 = weight.double().cpu()
    b64 = bias.double().cpu() if bias is not None else None
    use_rel = use_attn_bias or use_activation_bias
    for b, (start, n) in enumerate(_event_slices(seqlens, cu_seqlens, batch, length)):
        if n == 0:
            continue
        qe = _gather_event(q, b, start, n, packed).double().cpu() * s
        ke = _gather_event(k, b, start, n, packed).double().cpu()
        ve = _gather_event(v, b, start, n, packed).double().cpu()
        fe = _event_feats(feats, b, start, n, packed).cpu()
        for r0 in range(0, n, row_block):
            r1 = min(n, r0 + row_block)
            qi = qe[:, r0:r1]
            logits = qi @ ke.transpose(-1, -2)
            if use_rel:
                _, rel = _row_block_pair_terms(fe[r0:r1], fe, w64, b64)
                if use_attn_bias:
                    logits = logits + torch.einsum("hid,ijd->hij", qi, rel)
            blk_lse = torch.logsumexp(logits, -1)
            probs = torch.exp(logits - blk_lse[..., None])
            o = probs @ ve
            if use_activation_bias:
                o = o + torch.einsum("hij,ijd->hid", probs, rel)
            if packed:
                out[start + r0:start + r1] = o.transpose(0, 1)
                lse[start + r0:start + r1] = blk_lse.transpose(0, 1)
            else:
                out[b, :, r0:r1] = o
                lse[b, :, r0:r1] = blk_lse
    return out, lse


def backward_fp64_chunked(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    feats: Tensor,
    weight: Tensor,
    bias: Optional[Tensor],
    grad_out: Tensor,
    seqlens: Optional[Tensor] = None,
    scale: Optional[float] = None,
    use_attn_bias: bool = True,
    use_activation_bias: bool = True,
    cu_seqlens: Optional[Tensor] = None,
    row_block: int = 128,
    return_rowsum: bool = False,
):
    """Exact float64 gradients of the spec: (dq, dk, dv, dW, db[, rowsum]).

    Closed form of the reference definition, padding rows excluded (their
    upstream gradient is discarded, backward.py:526-532):

        s_ij  = qt_i.(k_j + [A] R_ij),        P = softmax_j(s)
        dP_ij = dO_i.(v_j + [V] R_ij),        D_i = sum_j P_ij dP_ij
        dS_ij = P_ij (dP_ij - D_i)
        dq_i  = scale * sum_j dS_ij (k_j + [A] R_ij)
        dk_j  = sum_i dS_ij qt_i,             dv_j = sum_i P_ij dO_i
        dR_ij = [A] dS_ij qt_i + [V] P_ij dO_i
        dW    = sum_ij dR_ij (x) E_ij,        db = sum_ij dR_ij

    `rowsum` (optional) is sum_j dS_ij per (row, head) -- zero in exact
    arithmetic, which the tests use as a closed-form check. dW/db are None
    when both bias flags are off (the projection is unused).
    """
    packed = cu_seqlens is not None
    head_dim = q.shape[-1]
    s = head_dim ** -0.5 if scale is None else scale
    batch = 0 if packed else q.shape[0]
    length = 0 if packed else q.shape[2]
    dq = torch.zeros(q.shape, dtype=torch.float64)
    dk = torch.zeros(q.shape, dtype=torch.float64)
    dv = torch.zeros(q.shape, dtype=torch.float64)
    rowsum = torch.zeros(q.shape[:-1], dtype=torch.float64)
    w64 = weight.double().cpu()
    b64 = bias.double().cpu() if bias is not None else None
    use_rel = use_attn_bias or use_activation_bias
    dW = torch.zeros_like(w64)
    db = torch.zeros(head_dim, dtype=torch.float64)
    for b, (start, n) in enumerate(_event_slices(seqlens, cu_seqlens, batch, length)):
        if n == 0:
            continue
        qe = _gather_event(q, b, start, n, packed).double().cpu() * s
        ke = _gather_event(k, b, start, n, packed).double().cpu()
        ve = _gather_event(v, b, start, n, packed).double().cpu()
        ge = _gather_event(grad_out, b, start, n, packed).double().cpu()
        fe = _event_feats(feats, b, start, n, packed).cpu()
        dke = torch.zeros_like(ke)
        dve = torch.zeros_like(ve)
        for r0 in range(0, n, row_block):
            r1 = min(n, r0 + row_block)
            qi, gi = qe[:, r0:r1], ge[:, r0:r1]
            logits = qi @ ke.transpose(-1, -2)
            dprob = gi @ ve.transpose(-1, -2)
            if use_rel:
                emb, rel = _row_block_pair_terms(fe[r0:r1], fe, w64, b64)
                if use_attn_bias:
                    logits = logits + torch.einsum("hid,ijd->hij", qi, rel)
                if use_activation_bias:
                    dprob = dprob + torch.einsum("hid,ijd->hij", gi, rel)
            probs = torch.softmax(logits, -1)
            dsum = (probs * dprob).sum(-1, keepdim=True)
            dlog = probs * (dprob - dsum)
            dqi = dlog @ ke
            if use_attn_bias:
                dqi = dqi + torch.einsum("hij,ijd->hid", dlog, rel)
            dke += dlog.transpose(-1, -2) @ qi
            dve += probs.transpose(-1, -2) @ gi
            if use_rel:
                drel = torch.zeros_like(rel)
                if use_attn_bias:
                    drel = drel + torch.einsum("hij,hid->ijd", dlog, qi)
                if use_activation_bias:
                    drel = drel + torch.einsum("hij,hid->ijd", probs, gi)
                dW += torch.einsum("ijd,ijc->dc", drel, emb)
                db += drel.sum((0, 1))
            rs = dlog.sum(-1)
            if packed:
                dq[start + r0:start + r1] = (dqi * s).transpose(0, 1)
                rowsum[start + r0:start + r1] = rs.transpose(0, 1)
            else:
                dq[b, :, r0:r1] = dqi * s
                rowsum[b, :, r0:r1] = rs
        if packed:
            dk[start:start + n] = dke.transpose(0, 1)
            dv[start:start + n] = dve.transpose(0, 1)
        else:
            dk[b, :, :n] = dke
            dv[b, :, :n] = dve
    out = (dq, dk, dv, dW if use_rel else None, db if use_rel else None)
    if return_rowsum:
        return out + (rowsum,)
    return out


def event_rows_fp64(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    feats: Tensor,
    weight: Tensor,
    bias: Optional[Tensor],
    grad_out: Optional[Tensor],
    rows: Tuple[int, int],
    scale: Optional[float] = None,
    use_attn_bias: bool = True,
    use_activation_bias: bool = True,
    dtype: torch.dtype = torch.float64,
) -> dict:
    """float64 terms of one event restricted to the query rows [r0, r1).

    q, k, v, grad_out: `[H, n, D]` (one event, valid tokens only); feats
    `[n, F]`. Returns the rows' `out`, `lse` (over the logits that include
    the `qt.b` term, like `attention_fp64_chunked`), `dq` and `rowsum`, and the
    contributions of those rows to `dk`, `dv` (`[H, n, D]`), `dW` and `db`:
    exactly the gradients of a call whose upstream gradient is zero outside
    the block, since a row with dO_i = 0 has dP_i = 0, D_i = 0 and dS_i = 0
    and adds nothing to any gradient (backward.py:3-32). The same
    closed-form terms as `backward_fp64_chunked` (reference.py:106-167,
    backward.py:155-168, 371-407, 600-622), evaluated for a row block only so
    that events of thousands of tokens stay cheap; `tests/test_oracle.py`
    checks the block sums against the whole-event evaluators.

    With `dtype` other than float64 every step runs in that dtype instead
    (pair angle and embedding in the feature dtype, as the eager definition
    does, reference.py:75-88): the eager evaluation whose error is the
    yardstick of the "2x eager" rule (reference test_gpu.py:133-169).
    """
    r0, r1 = rows
    head_dim = q.shape[-1]
    s = head_dim ** -0.5 if scale is None else scale
    qe = q.to(dtype).cpu() * s
    ke = k.to(dtype).cpu()
    ve = v.to(dtype).cpu()
    fe = feats.to(dtype).cpu()
    w64 = weight.to(dtype).cpu()
    b64 = bias.to(dtype).cpu() if bias is not None else None
    use_rel = use_attn_bias or use_activation_bias
    qi = qe[:, r0:r1]
    logits = qi @ ke.transpose(-1, -2)
    emb = rel = None
    if use_rel:
        if dtype == torch.float64:
            emb, rel = _row_block_pair_terms(fe[r0:r1], fe, w64, b64)
        else:
            emb = embed_angle(pair_angle_rect(fe[r0:r1][None], fe[None])[0], w64.shape[1]).to(dtype)
            rel = emb @ w64.t()
            if b64 is not None:
                rel = rel + b64
        if use_attn_bias:
            logits = logits + torch.einsum("hid,ijd->hij", qi, rel)
    lse = torch.logsumexp(logits, -1)
    probs = torch.exp(logits - lse[..., None])
    out = probs @ ve
    if use_activation_bias:
        out = out + torch.einsum("hij,ijd->hid", probs, rel)
    res = {"out": out, "lse": lse}
    if grad_out is None:
        return res
    gi = grad_out.to(dtype).cpu()[:, r0:r1]
    dprob = gi @ ve.transpose(-1, -2)
    if use_activation_bias:
        dprob = dprob + torch.einsum("hid,ijd->hij", gi, rel)
    dsum = (probs * dprob).sum(-1, keepdim=True)
    dlog = probs * (dprob - dsum)
    dqi = dlog @ ke
    if use_attn_bias:
        dqi = dqi + torch.einsum("hij,ijd->hid", dlog, rel)
    res["dq"] = dqi * s
    res["rowsum"] = dlog.sum(-1)
    res["dk"] = dlog.transpose(-1, -2) @ qi
    res["dv"] = probs.transpose(-1, -2) @ gi
    if use_rel:
        drel = torch.zeros_like(rel)
        if use_attn_bias:
            drel = drel + torch.einsum("hij,hid->ijd", dlog, qi)
        if use_activation_bias:
            drel = drel + torch.einsum("hij,hid->ijd", probs, gi)
        res["dW"] = torch.einsum("ijd,ijc->dc", drel, emb)
        res["db"] = drel.sum((0, 1))
    else:
        res["dW"] = res["db"] = None
    return res
