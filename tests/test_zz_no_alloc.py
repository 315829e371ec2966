"""fst_forward_noalloc: the allocation-free forward entry point (C ABI).

It has no reference counterpart; it is for callers that cannot allocate
device memory. Checked through the C ABI against fst_forward (same kernels
and work list, so bitwise equal), on two calls in a row, the second with a
smaller input, in the padded and packed layouts; plus its size limit.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from flash_spacetime_amd import _lib
    from flash_spacetime_amd.forward import _Prepared

DEV = "cuda"


def _case(batch, length, seed, packed):
    gen = torch.Generator().manual_seed(seed)
    H, D, C = 12, 32, 16
    lens = torch.randint(1, length + 1, (batch,), generator=gen)
    lens[0] = length
    if packed:
        total = int(lens.sum())
        q, k, v = (torch.randn(total, H, D, generator=gen).to(DEV, torch.bfloat16) for _ in range(3))
        feats = torch.randn(total, 4, generator=gen).to(DEV)
        cu = torch.cat([torch.zeros(1, dtype=torch.long), lens.cumsum(0)]).to(DEV, torch.int32)
        seqlens = None
    else:
        q, k, v = (torch.randn(batch, H, length, D, generator=gen).to(DEV, torch.bfloat16) for _ in range(3))
        feats = torch.randn(batch, length, 4, generator=gen).to(DEV)
        cu = None
        seqlens = lens.to(DEV, torch.int32)
    w = (torch.randn(D, C, generator=gen) / 4).to(DEV)
    b = (torch.randn(D, generator=gen) * 0.02).to(DEV)
    return _Prepared(q, k, v, feats, w, b, seqlens, None, True, True, cu)


def _args(prep):
    P = _lib.ptr
    return (P(prep.q), P(prep.k), P(prep.v), P(prep.pos4), P(prep.weight), P(prep.bias), P(prep.lens), prep.scale)


def _reference_forward(lib, prep):
    dims = prep.dims()
    out, lse = torch.empty_like(prep.q), prep.empty_vec()
    nbytes = lib.fst_forward_workspace_bytes(*dims)
    ws = torch.empty(nbytes, device=DEV, dtype=torch.uint8)
    rc = lib.fst_forward(*dims, *_args(prep), _lib.ptr(out), _lib.ptr(lse), _lib.ptr(ws), nbytes,
                         _lib.stream_handle(prep.device))
    _lib.check(rc, "fst_forward")
    return out, lse


def _noalloc_forward(lib, prep):
    out, lse = torch.empty_like(prep.q), prep.empty_vec()
    rc = lib.fst_forward_noalloc(*prep.dims(), *_args(prep), _lib.ptr(out), _lib.ptr(lse),
                                 _lib.stream_handle(prep.device))
    _lib.check(rc, "fst_forward_noalloc")
    return out, lse


@pytest.mark.parametrize("packed", [False, True], ids=["padded", "packed"])
def test_noalloc_forward_equals_forward(packed):
    lib = _lib.load()
    for batch, length, seed in ((64, 300, 1), (5, 70, 2)):  # the second call is smaller
        print(f"noalloc forward: packed={packed} B={batch} L={length}", flush=True)
        prep = _case(batch, length, seed, packed)
        want_out, want_lse = _reference_forward(lib, prep)
        got_out, got_lse = _noalloc_forward(lib, prep)
        torch.cuda.synchronize()
        assert torch.equal(got_out, want_out)
        assert torch.equal(got_lse, want_lse)


def test_noalloc_forward_rejects_too_many_events():
    lib = _lib.load()
    rc = lib.fst_forward_noalloc(_lib.FST_BF16, 3, 65537, 12, 16, 0, 32, 16, *([None] * 7), 1.0, None, None,
                                 _lib.stream_handle(torch.device(DEV)))
    assert rc == _lib.FST_EUNSUPPORTED and "65536" in _lib.last_error()


def test_noalloc_forward_under_graph_capture():
    """Captured after one eager call: every replay bitwise equal to fst_forward,
    with eager work between the replays, and a second, smaller captured call
    after the first graph's replays."""
    lib = _lib.load()
    for batch, length, seed in ((32, 200, 3), (4, 40, 4)):
        prep = _case(batch, length, seed, False)
        want_out, want_lse = _reference_forward(lib, prep)
        _noalloc_forward(lib, prep)  # eager warm-up on this stream
        torch.cuda.synchronize()
        out, lse = torch.empty_like(prep.q), prep.empty_vec()
        graph = torch.cuda.CUDAGraph()
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            with torch.cuda.graph(graph, stream=stream):
                rc = lib.fst_forward_noalloc(*prep.dims(), *_args(prep), _lib.ptr(out), _lib.ptr(lse),
                                             _lib.stream_handle(prep.device))
        torch.cuda.current_stream().wait_stream(stream)
        _lib.check(rc, "fst_forward_noalloc (captured)")
        for rep in range(3):
            out.zero_()
            lse.fill_(float("nan"))
            graph.replay()
            torch.cuda.synchronize()
            print(f"replay {rep}: B={batch} L={length}", flush=True)
            assert torch.equal(out, want_out) and torch.equal(lse, want_lse)
            _reference_forward(lib, _case(3, 30, 9, False))  # eager work between replays
            torch.cuda.synchronize()


_FIRST_CALL_CAPTURED = r"""
import sys, torch
sys.path.insert(0, sys.argv[1])
from tests.test_zz_no_alloc import _case, _args, _reference_forward
from flash_spacetime_amd import _lib
lib = _lib.load()
prep = _case(16, 100, 5, False)
want_out, want_lse = _reference_forward(lib, prep)
torch.cuda.synchronize()
out, lse = torch.empty_like(prep.q), prep.empty_vec()
graph = torch.cuda.CUDAGraph()
stream = torch.cuda.Stream()
stream.wait_stream(torch.cuda.current_stream())
with torch.cuda.stream(stream):
    with torch.cuda.graph(graph, stream=stream):
        rc = lib.fst_forward_noalloc(*prep.dims(), *_args(prep), _lib.ptr(out), _lib.ptr(lse),
                                     _lib.stream_handle(prep.device))
torch.cuda.current_stream().wait_stream(stream)
_lib.check(rc, "first fst_forward_noalloc call, captured")
for _ in range(2):
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, want_out) and torch.equal(lse, want_lse)
print("first captured call ok", flush=True)
"""


def test_noalloc_forward_first_call_captured():
    """The first call on a device (where the scratch address is resolved) made
    under graph capture, in a fresh process of its own."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    res = subprocess.run([sys.executable, "-c", _FIRST_CALL_CAPTURED, root], capture_output=True, text=True,
                         timeout=100)
    print(res.stdout[-2000:], res.stderr[-2000:], flush=True)
    assert res.returncode == 0 and "first captured call ok" in res.stdout
