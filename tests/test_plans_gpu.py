"""GPU tests of the kernel plans (FST_PLAN_* bits) and the measured tuner.

Parity rule for the variants. The occupancy, wave, K/V-staging and
tile-height groups compute every output row with the same arithmetic, so
for every supported combination of them out, lse, dq, dk, dv and the dS row
sums must equal the static plan's bit for bit, and dW and db (whose fp32
per-tile partials another wave or tile layout adds in another order) agree
to fp32 rounding. The key-chunk groups move the online softmax's rescaling
points and the order of the key sums, and the float32 rows kernel's pass
group forms D online or in a first pass: a combination with such a bit is
held to the float64 oracle at the dtype's tolerance (bf16 2e-2, float32
1e-4 relative). The tuner, switched on, must pick plans the shape offers (or
keep the static one) and leave every result as that rule allows.
"""

import itertools

import pytest
import torch

import oracle
from tests._cases import rel_err

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from flash_spacetime_amd import (
        _lib, flash_spacetime_attention, flash_spacetime_backward, flash_spacetime_forward, tune,
    )

DEV = "cuda"
BF, F32 = 0, 1
TOL = {BF: 2e-2, F32: 1e-4}
# Groups whose variants change the order of the arithmetic: FST_PLAN_FWD_KC*,
# FST_PLAN_BWD_KC*, FST_PLAN_BWD_PASS* (D formed online or in a first pass).
KC_BITS = (1 << 17) | (1 << 18) | (1 << 25) | (1 << 26) | (1 << 27) | (1 << 28)

# (dtype, heads, dim, channels, lengths, packed, bias flags)
SHAPES = [
    (BF, 12, 32, 16, [80, 33, 1], False, (True, True)),    # cfg2's head layout
    (BF, 12, 32, 16, [80, 33, 1], False, (True, False)),   # flags read at run time
    (BF, 4, 16, 32, [50, 17, 3], True, (True, True)),
    (BF, 16, 16, 16, [64, 40], False, (False, True)),
    (BF, 8, 48, 16, [70, 9, 33], True, (True, True)),
    (BF, 8, 64, 64, [48, 21], False, (True, True)),        # one variant of each kernel
    (BF, 12, 64, 32, [70, 40], False, (True, True)),       # K / V in LDS with two 32-feature parts
    (BF, 4, 32, 16, [90, 20], True, (True, True)),         # eight waves with four owning no head
    (F32, 4, 16, 16, [70, 33], False, (True, True)),
    (F32, 12, 32, 16, [80, 33, 1], True, (True, True)),
    (F32, 8, 64, 64, [48, 21], False, (True, True)),
    (F32, 16, 32, 16, [70, 33], True, (True, True)),       # eight waves, two heads each
    (F32, 8, 32, 16, [90, 17, 1], False, (True, False)),   # eight waves, lanes sharing an embedding
    (F32, 7, 32, 16, [70, 33], False, (True, True)),       # eight waves, one owning only a padded head
    (F32, 13, 16, 32, [60, 21], True, (False, True)),      # eight waves over 16 padded heads
    (F32, 4, 16, 48, [57, 30, 1], False, (True, True)),    # D = 16 with wide C: every variant
    (F32, 6, 16, 64, [45, 20], True, (True, True)),
    (F32, 16, 16, 48, [40, 17], False, (True, False)),
]

FWD_GROUPS = [(1 << 8, 1 << 9), (1 << 17, 1 << 18), (1 << 19, 1 << 20, 1 << 21, 1 << 29)]
BWD_GROUPS = [(1 << 10, 1 << 11, 1 << 14), (1 << 15, 1 << 16), (1 << 12, 1 << 13),
              (1 << 22, 1 << 23, 1 << 24, 1 << 30), (1 << 25, 1 << 26), (1 << 27, 1 << 28)]


def _inputs(dtype, heads, dim, chans, lens, packed, seed):
    gen = torch.Generator().manual_seed(seed)
    rn = lambda *s: torch.randn(*s, generator=gen, dtype=torch.float64)  # noqa: E731
    tdt = torch.bfloat16 if dtype == BF else torch.float32
    if packed:
        total = sum(lens)
        shape, fshape = (total, heads, dim), (total,)
        cu = torch.zeros(len(lens) + 1, dtype=torch.int32)
        cu[1:] = torch.cumsum(torch.tensor(lens), 0)
        sl, cu = None, cu
    else:
        length = max(lens)
        shape, fshape = (len(lens), heads, length, dim), (len(lens), length)
        sl, cu = torch.tensor(lens, dtype=torch.int32), None
    q, k, v, do = (rn(*shape).to(tdt) for _ in range(4))
    feats = rn(*fshape, 4).float()  # randn positions, the reference tests' distribution
    w = (rn(dim, chans) / chans ** 0.5).float()
    b = (rn(dim) * 0.02).float()
    return q, k, v, do, feats, w, b, sl, cu


def _run(args, flags, with_out=False):
    q, k, v, do, feats, w, b, sl, cu = (x.to(DEV) if x is not None else None for x in args)
    kw = dict(use_attn_bias=flags[0], use_activation_bias=flags[1], cu_seqlens=cu)
    out, lse = flash_spacetime_forward(q, k, v, feats, w, b, sl, **kw)
    rowsum = torch.zeros_like(lse)
    grads = flash_spacetime_backward(q, k, v, feats, w, b, sl, lse, do, rowsum=rowsum,
                                     out=out if with_out else None, **kw)
    torch.cuda.synchronize()
    return out, lse, rowsum, grads


def _oracle(args, flags, packed):
    q, k, v, do, feats, w, b, sl, cu = args
    d = lambda t: t.double()  # noqa: E731
    kw = dict(use_attn_bias=flags[0], use_activation_bias=flags[1], cu_seqlens=cu)
    lens = None if packed else sl.long()
    out, _ = oracle.attention_fp64_chunked(d(q), d(k), d(v), d(feats), d(w), d(b), lens, **kw)
    dor = d(do)
    if not packed:
        dor = dor * oracle.valid_row_mask(q.shape[0], q.shape[2], lens)[:, None, :, None]
        out = out * oracle.valid_row_mask(q.shape[0], q.shape[2], lens)[:, None, :, None]
    grads = oracle.backward_fp64_chunked(d(q), d(k), d(v), d(feats), d(w), d(b), dor, lens, **kw)
    return out, list(grads)


def _full_combos(dtype, heads, dim, chans, groups):
    """Every supported plan with one bit in each group the shape offers."""
    mask = tune.plans(dtype, heads, dim, chans)
    choices = [[bit for bit in g if mask & bit] or [0] for g in groups]
    plans = {sum(c) for c in itertools.product(*choices)} - {0}
    return sorted(p for p in plans if tune.plan_supported(dtype, heads, dim, chans, p))


def _same(got, base):
    """out, lse, rowsum, dq, dk, dv bit for bit; dW, db to fp32 rounding."""
    if not (torch.equal(got[0], base[0]) and torch.equal(got[1], base[1]) and torch.equal(got[2], base[2])):
        return False
    if not all(torch.equal(g, r) for g, r in zip(got[3][:3], base[3][:3])):
        return False
    return all(r is None or rel_err(g, r) <= 1e-5 for g, r in zip(got[3][3:], base[3][3:]))


@pytest.mark.parametrize("with_out", [False, True], ids=["online_d", "reference_d"])
@pytest.mark.parametrize("case", range(len(SHAPES)))
def test_every_plan_matches_the_static_plan(case, with_out):
    """Fully specified plans (one bit in every offered group) of one kernel
    family, classed by their key-chunk bits: plans of one class agree bit for
    bit, each class is within the dtype's tolerance of the float64 oracle,
    and the static plan is bit for bit one of the classes. with_out: the
    backward is given the forward's output (the bf16 rows kernel's
    reference D; float32 ignores it)."""
    dtype, heads, dim, chans, lens, packed, flags = SHAPES[case]
    if with_out and dtype == F32:
        pytest.skip("float32 kernels do not read the output")
    args = _inputs(dtype, heads, dim, chans, lens, packed, 100 + case)
    tune.set_autotune(False)
    base = _run(args, flags, with_out)
    ref = _oracle(args, flags, packed)
    valid = None if packed else \
        oracle.valid_row_mask(len(lens), max(lens), torch.tensor(lens))[:, None, :, None].to(DEV)
    for groups in (FWD_GROUPS, BWD_GROUPS):
        classes = {}
        for plan in _full_combos(dtype, heads, dim, chans, groups):
            print(f"plan {tune.plan_names(plan)}", flush=True)
            with tune.fixed_plan(plan):
                got = _run(args, flags, with_out)
            kc = plan & KC_BITS
            if kc in classes:
                assert _same(got, classes[kc][1]), f"{tune.plan_names(plan)} vs {tune.plan_names(classes[kc][0])}"
                continue
            classes[kc] = (plan, got)
            kern = [got[0] if valid is None else got[0] * valid] + list(got[3])
            for name, a, e in zip(["out", "dq", "dk", "dv", "dW", "db"], kern, [ref[0]] + ref[1]):
                if e is None or (name == "db" and not flags[1]):
                    continue
                err = rel_err(a, e)
                assert err <= TOL[dtype], f"{tune.plan_names(plan)}: {name} relative error {err:.3e}"
        assert classes
        assert any(_same(base, got) for _, got in classes.values()), "the static plan matches no class"


@pytest.mark.parametrize("dtype", [BF, F32], ids=["bf16", "fp32"])
def test_tile_arguments_run_their_variant(dtype):
    """The reference launchers' block_m / block_n / num_warps select the
    variant tune.plan_from_tiles names: the results are those of that plan."""
    heads, dim, chans, lens = (12, 32, 16, [80, 33]) if dtype == BF else (4, 16, 16, [70, 33])
    args = _inputs(dtype, heads, dim, chans, lens, False, 7)
    q, k, v, do, feats, w, b, sl, _ = (x.to(DEV) if x is not None else None for x in args)
    tiles = dict(block_m=32, block_n=32, num_warps=4)
    out, lse = flash_spacetime_forward(q, k, v, feats, w, b, sl, **tiles)
    grads = flash_spacetime_backward(q, k, v, feats, w, b, sl, lse, do, **tiles)
    fplan = tune.plan_from_tiles(dtype, heads, dim, chans, "fwd", **tiles)
    bplan = tune.plan_from_tiles(dtype, heads, dim, chans, "bwd", **tiles)
    assert fplan and bplan
    with tune.fixed_plan(fplan | bplan):
        out2, lse2 = flash_spacetime_forward(q, k, v, feats, w, b, sl)
        grads2 = flash_spacetime_backward(q, k, v, feats, w, b, sl, lse2, do)
    torch.cuda.synchronize()
    assert torch.equal(out, out2) and torch.equal(lse, lse2)
    for g, r in zip(grads, grads2):
        assert torch.equal(g, r)


def test_unoffered_plan_is_refused():
    args = _inputs(BF, 8, 64, 64, [48, 21], False, 7)
    with tune.fixed_plan(_lib.FST_PLAN_FWD_OCC3):
        with pytest.raises(ValueError, match="plan"):
            _run(args, (True, True))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_autotune_picks_offered_plans_and_keeps_results(dtype):
    # float32 also covers the tuner's tile-height groups, whose candidates
    # each need a work list of their own rows per workgroup.
    heads, dim, chans = 12, 32, 16
    gen = torch.Generator().manual_seed(5)
    lens = torch.randint(16, 257, (24,), generator=gen)
    length = 256
    rn = lambda *s: torch.randn(*s, generator=gen)  # noqa: E731
    q, k, v, do = (rn(24, heads, length, dim).to(DEV, dtype) for _ in range(4))
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
    kinds = sorted(k[2] for k in picked)
    assert kinds == ["bwd", "fwd"], picked
    fp32 = dtype == torch.float32
    mask = tune.plans(_lib.FST_F32 if fp32 else _lib.FST_BF16, heads, dim, chans)
    for key, plan in picked.items():
        assert plan & ~mask == 0, (key, hex(plan))  # 0: the static choice kept
        print(key, tune.plan_names(plan), flush=True)
    kc = any(plan & KC_BITS for plan in picked.values())
    for run in (first, second):
        # a key-chunk variant (or, in float32, another pass count) agrees to
        # rounding, every other one exactly
        if fp32:
            cmp = lambda a, b: rel_err(a, b) <= 1e-5  # noqa: E731
        else:
            cmp = (lambda a, b: rel_err(a, b) <= 2e-2) if kc else torch.equal
        assert cmp(run[0], ref[0])
        for g, r in zip(run[1], ref[1]):
            assert cmp(g, r)
