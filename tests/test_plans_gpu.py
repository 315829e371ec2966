"""GPU tests of the kernel plans (FST_PLAN_* bits) and the measured tuner.

Every compiled variant of a kernel computes each output row with the same
arithmetic, so for every plan a shape offers, out, lse, dq, dk, dv and the
dS row sums must equal the static plan's bitwise; dW and db, whose fp32
per-tile partials the eight-wave rows kernel combines in another order,
agree to fp32 rounding. The tuner, switched on, must pick plans the shape
offers (or keep the static one) and leave every result as the static plan
computes it.
"""

import itertools

import pytest
import torch

from tests._cases import rel_err

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from flash_spacetime_amd import (
        _lib, flash_spacetime_attention, flash_spacetime_backward, flash_spacetime_forward, tune,
    )

DEV = "cuda"

# (heads, dim, channels, lengths, packed, bias flags)
SHAPES = [
    (12, 32, 16, [80, 33, 1], False, (True, True)),    # cfg2's head layout
    (12, 32, 16, [80, 33, 1], False, (True, False)),   # flags read at run time
    (4, 16, 32, [50, 17, 3], True, (True, True)),
    (16, 16, 16, [64, 40], False, (False, True)),
    (8, 48, 16, [70, 9, 33], True, (True, True)),
    (8, 64, 64, [48, 21], False, (True, True)),        # one variant of each kernel
]


def _inputs(heads, dim, chans, lens, packed, seed):
    gen = torch.Generator().manual_seed(seed)
    rn = lambda *s: torch.randn(*s, generator=gen)  # noqa: E731
    if packed:
        total = sum(lens)
        shape, fshape = (total, heads, dim), (total,)
        cu = torch.zeros(len(lens) + 1, dtype=torch.int32)
        cu[1:] = torch.cumsum(torch.tensor(lens), 0)
        sl, cu = None, cu.to(DEV)
    else:
        length = max(lens)
        shape, fshape = (len(lens), heads, length, dim), (len(lens), length)
        sl, cu = torch.tensor(lens, dtype=torch.int32, device=DEV), None
    q, k, v, do = (rn(*shape).to(DEV, torch.bfloat16) for _ in range(4))
    feats = torch.cat([(torch.rand(*fshape, 3, generator=gen) - 0.5) * 1000,
                       torch.rand(*fshape, 1, generator=gen) * 2e4], -1).to(DEV)
    w = (rn(dim, chans) / chans ** 0.5).to(DEV)
    b = (rn(dim) * 0.02).to(DEV)
    return q, k, v, do, feats, w, b, sl, cu


def _run(args, flags):
    q, k, v, do, feats, w, b, sl, cu = args
    kw = dict(use_attn_bias=flags[0], use_activation_bias=flags[1], cu_seqlens=cu)
    out, lse = flash_spacetime_forward(q, k, v, feats, w, b, sl, **kw)
    rowsum = torch.zeros_like(lse)
    grads = flash_spacetime_backward(q, k, v, feats, w, b, sl, lse, do, rowsum=rowsum, **kw)
    torch.cuda.synchronize()
    return out, lse, rowsum, grads


def _plans_of(mask):
    pick = lambda bits: [x for x in bits if mask & x]  # noqa: E731
    fwd = pick((_lib.FST_PLAN_FWD_OCC2, _lib.FST_PLAN_FWD_OCC3))
    rows = pick((_lib.FST_PLAN_ROWS_W4, _lib.FST_PLAN_ROWS_W8))
    cols = pick((_lib.FST_PLAN_COLS_OCC2, _lib.FST_PLAN_COLS_OCC3))
    return [f | r | c for f, r, c in itertools.product(fwd, rows, cols)]


@pytest.mark.parametrize("case", range(len(SHAPES)))
def test_every_plan_matches_the_static_plan(case):
    heads, dim, chans, lens, packed, flags = SHAPES[case]
    args = _inputs(heads, dim, chans, lens, packed, 100 + case)
    tune.set_autotune(False)
    base = _run(args, flags)
    mask = tune.plans(_lib.FST_BF16, heads, dim, chans)
    combos = _plans_of(mask)
    assert combos, hex(mask)
    for plan in combos:
        print(f"plan {tune.plan_names(plan)}", flush=True)
        with tune.fixed_plan(plan):
            got = _run(args, flags)
        assert torch.equal(got[0], base[0]) and torch.equal(got[1], base[1]), tune.plan_names(plan)
        assert torch.equal(got[2], base[2]), tune.plan_names(plan)
        for g, r in zip(got[3][:3], base[3][:3]):
            assert torch.equal(g, r), tune.plan_names(plan)
        assert rel_err(got[3][3], base[3][3]) <= 1e-5 and rel_err(got[3][4], base[3][4]) <= 1e-5


def test_unoffered_plan_is_refused():
    args = _inputs(8, 64, 64, [48, 21], False, 7)
    with tune.fixed_plan(_lib.FST_PLAN_FWD_OCC3):
        with pytest.raises(ValueError, match="plan"):
            _run(args, (True, True))


def test_autotune_picks_offered_plans_and_keeps_results():
    heads, dim, chans = 12, 32, 16
    gen = torch.Generator().manual_seed(5)
    lens = torch.randint(16, 257, (24,), generator=gen)
    length = 256
    rn = lambda *s: torch.randn(*s, generator=gen)  # noqa: E731
    q, k, v, do = (rn(24, heads, length, dim).to(DEV, torch.bfloat16) for _ in range(4))
    feats = torch.cat([(torch.rand(24, length, 3, generator=gen) - 0.5) * 1000,
                       torch.rand(24, length, 1, generator=gen) * 2e4], -1).to(DEV)
    w = (rn(dim, chans) / 4).to(DEV)
    b = (rn(dim) * 0.02).to(DEV)
    sl = lens.to(DEV, torch.int32)

    def step():
        leaves = [x.detach().clone().requires_grad_(True) for x in (q, k, v)]
        out = flash_spacetime_attention(*leaves, feats, w, b, sl)
        out.backward(do)
        torch.cuda.synchronize()
        return out.detach(), [x.grad for x in leaves]

    tune.clear()
    tune.set_autotune(False)
    ref = step()
    try:
        tune.set_autotune(True)
        first = step()
        picked = tune.chosen()
        second = step()
        assert tune.chosen() == picked  # the second call of the shape reuses the choice
    finally:
        tune.set_autotune(False)
        tune.clear()
    kinds = sorted(k[0] for k in picked)
    assert kinds == ["bwd", "fwd"], picked
    mask = tune.plans(_lib.FST_BF16, heads, dim, chans)
    for key, plan in picked.items():
        assert plan & ~mask == 0, (key, hex(plan))  # 0: the static choice kept
        print(key, tune.plan_names(plan), flush=True)
    for run in (first, second):
        assert torch.equal(run[0], ref[0])
        for g, r in zip(run[1], ref[1]):
            assert torch.equal(g, r)
