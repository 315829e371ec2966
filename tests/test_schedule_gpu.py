"""GPU tests of the tile kernels' work schedules.

The bf16 kernels deal tiles to the XCDs longest event first: padded events
in snake order of a length sort, packed tiles in groups of eight over the
sorted tile list. Past 8192 events the sort falls back to event order. The
schedule decides only which workgroup computes a tile: every tile's rows and
every per-tile output slot are the same, so results must be bitwise
independent of it. These tests run more events than the sort handles, with
empty events among them, and compare against the same events in two
smaller calls (each sorted) — out, dq, dk, dv bitwise; dW and db, whose
per-tile partials are summed over different sets, to fp32 rounding.
"""

import pytest
import torch

from tests._cases import rel_err

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from flash_spacetime_amd import flash_spacetime_attention, flash_spacetime_attention_varlen

DEV = "cuda"
N_EVENTS = 9000  # more than the 8192 events the length sort handles


def _leaves(*xs):
    return [x.detach().clone().requires_grad_(True) for x in xs]


def _packed_inputs(lens, heads, dim, chans, seed):
    gen = torch.Generator().manual_seed(seed)
    total = int(sum(lens))
    rn = lambda *s: torch.randn(*s, generator=gen)
    q, k, v, do = (rn(total, heads, dim).to(DEV, torch.bfloat16) for _ in range(4))
    feats = torch.cat([(torch.rand(total, 3, generator=gen) - 0.5) * 1000,
                       torch.rand(total, 1, generator=gen) * 2e4], -1).to(DEV)
    w = (rn(dim, chans) / chans ** 0.5).to(DEV)
    b = (rn(dim) * 0.02).to(DEV)
    return q, k, v, do, feats, w, b


def _cu(lens):
    cu = torch.zeros(len(lens) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lens, dtype=torch.int64), 0).to(torch.int32)
    return cu.to(DEV)


def _run_packed(q, k, v, do, feats, w, b, lens):
    leaves = _leaves(q, k, v, w, b)
    out = flash_spacetime_attention_varlen(*leaves[:3], feats, leaves[3], leaves[4], _cu(lens))
    out.backward(do)
    return out.detach(), [x.grad for x in leaves]


def test_packed_many_events_match_split_calls():
    gen = torch.Generator().manual_seed(71)
    lens = torch.randint(0, 40, (N_EVENTS,), generator=gen)
    lens[::97] = 0
    lens[5] = 600  # one long event among many short ones
    lens = lens.tolist()
    q, k, v, do, feats, w, b = _packed_inputs(lens, 4, 32, 16, 72)
    out, grads = _run_packed(q, k, v, do, feats, w, b, lens)
    half = N_EVENTS // 2
    t0 = sum(lens[:half])
    parts = [(lens[:half], slice(0, t0)), (lens[half:], slice(t0, None))]
    outs, gq, gk, gv, gw, gb = [], [], [], [], 0, 0
    for pl, sl in parts:
        o, g = _run_packed(q[sl], k[sl], v[sl], do[sl], feats[sl], w, b, pl)
        outs.append(o)
        gq.append(g[0])
        gk.append(g[1])
        gv.append(g[2])
        gw = gw + g[3]
        gb = gb + g[4]
    assert torch.equal(out, torch.cat(outs))
    for full, split in ((grads[0], gq), (grads[1], gk), (grads[2], gv)):
        assert torch.equal(full, torch.cat(split))
    assert rel_err(grads[3], gw) <= 1e-5 and rel_err(grads[4], gb) <= 1e-5


def test_padded_many_events_match_split_calls():
    gen = torch.Generator().manual_seed(73)
    length, heads, dim, chans = 24, 2, 16, 16
    lens = torch.randint(0, length + 1, (N_EVENTS,), generator=gen)
    lens[::89] = 0
    rn = lambda *s: torch.randn(*s, generator=gen)
    q, k, v, do = (rn(N_EVENTS, heads, length, dim).to(DEV, torch.bfloat16) for _ in range(4))
    feats = torch.cat([(torch.rand(N_EVENTS, length, 3, generator=gen) - 0.5) * 1000,
                       torch.rand(N_EVENTS, length, 1, generator=gen) * 2e4], -1).to(DEV)
    w = (rn(dim, chans) / chans ** 0.5).to(DEV)
    b = (rn(dim) * 0.02).to(DEV)
    sl = lens.to(DEV, torch.int32)

    def run(lo, hi):
        leaves = _leaves(q[lo:hi], k[lo:hi], v[lo:hi], w, b)
        out = flash_spacetime_attention(*leaves[:3], feats[lo:hi], leaves[3], leaves[4], sl[lo:hi])
        out.backward(do[lo:hi])
        return out.detach(), [x.grad for x in leaves]

    out, grads = run(0, N_EVENTS)
    half = N_EVENTS // 2
    (o1, g1), (o2, g2) = run(0, half), run(half, N_EVENTS)
    assert torch.equal(out, torch.cat([o1, o2]))
    for i in range(3):
        assert torch.equal(grads[i], torch.cat([g1[i], g2[i]]))
    assert rel_err(grads[3], g1[3] + g2[3]) <= 1e-5 and rel_err(grads[4], g1[4] + g2[4]) <= 1e-5
    # Padding rows (and whole empty events) are exact zeros.
    valid = torch.arange(length, device=DEV)[None, :] < sl[:, None]
    vm = valid[:, None, :, None].expand(out.shape)
    assert (out[~vm] == 0).all() and all((g[~vm] == 0).all() for g in grads[:3])


def test_packed_sorted_schedule_is_deterministic():
    gen = torch.Generator().manual_seed(75)
    lens = torch.exp(4.0 + torch.randn(300, generator=gen, dtype=torch.float64)).round().clamp(0, 1500).long()
    lens = lens.tolist()
    q, k, v, do, feats, w, b = _packed_inputs(lens, 6, 32, 16, 76)
    a = _run_packed(q, k, v, do, feats, w, b, lens)
    c = _run_packed(q, k, v, do, feats, w, b, lens)
    assert torch.equal(a[0], c[0]) and all(torch.equal(x, y) for x, y in zip(a[1], c[1]))


@pytest.mark.parametrize("batch", [1, 5, 256, 1024, 1025, 2048, 2049, 3000, 4096, 4097, 8192, 9000])
def test_event_sort_order(batch):
    """The forward work list's event order (workspace ints B+1 .. 2B): events
    by decreasing length, ties by index, up to 8192 events (rank sort up to
    1024, bitonic above); the identity past that."""
    from flash_spacetime_amd import _lib

    lib = _lib.load()
    gen = torch.Generator().manual_seed(batch)
    length, heads, dim, chans = 8, 1, 16, 16
    lens = torch.randint(0, length + 1, (batch,), generator=gen, dtype=torch.int32)
    q = torch.zeros(batch, heads, length, dim, device=DEV, dtype=torch.bfloat16)
    pos4 = torch.zeros(batch, length, 4, device=DEV)
    w = torch.zeros(dim, chans, device=DEV)
    out, lse = torch.empty_like(q), torch.empty(batch, heads, length, device=DEV)
    dims = (_lib.FST_BF16, 3, batch, heads, length, 0, dim, chans)
    ws_bytes = lib.fst_forward_workspace_bytes(*dims)
    ws = torch.zeros(ws_bytes // 4, device=DEV, dtype=torch.int32)
    rc = lib.fst_forward_phases(_lib.FST_PHASE_WORKLIST, *dims, q.data_ptr(), q.data_ptr(), q.data_ptr(),
                                pos4.data_ptr(), w.data_ptr(), None, lens.to(DEV).data_ptr(), 1.0,
                                out.data_ptr(), lse.data_ptr(), ws.data_ptr(), ws_bytes,
                                torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "work list")
    torch.cuda.synchronize()
    perm = ws[batch + 1: 2 * batch + 1].cpu().tolist()
    if batch <= 8192:
        want = sorted(range(batch), key=lambda i: (-int(lens[i]), i))
    else:
        want = list(range(batch))
    assert perm == want
