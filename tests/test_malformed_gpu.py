"""Malformed packed offsets on the GPU: the fixed work list keeps every access
inside the tensors and the workspace, and the kernels write NaN into the
rows they cover instead of results (include/flash_spacetime.h).

cu_seqlens = [0, 800, 0, 1600] with T = 1600 describes overlapping events;
before the work list sanitised offsets, the backward's per-tile slots could
be overrun (50 + 100 tiles against ceil(1600 / 16) + 3 = 103 slots). On the
sanitised offsets [0, 800, 800, 1600] the events hold 100 tiles. The case is
within every bound (checked on the CPU in tests/test_abi_cpu.py), so this is
an ordinary regression test of the fixed code.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from flash_spacetime_amd import flash_spacetime_backward, flash_spacetime_forward

DEV = "cuda"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_overlapping_cu_seqlens_give_nan_rows(dtype):
    gen = torch.Generator().manual_seed(7)
    total, H, D, C = 1600, 12, 32, 16
    q, k, v, do = (torch.randn(total, H, D, generator=gen).to(DEV, dtype) for _ in range(4))
    feats = torch.randn(total, 4, generator=gen).to(DEV)
    w = (torch.randn(D, C, generator=gen) / 4).to(DEV)
    b = (torch.randn(D, generator=gen) * 0.02).to(DEV)
    cu = torch.tensor([0, 800, 0, 1600], dtype=torch.int32, device=DEV)
    print(f"malformed cu_seqlens {cu.tolist()}, dtype {dtype}", flush=True)
    out, lse = flash_spacetime_forward(q, k, v, feats, w, b, None, cu_seqlens=cu)
    rowsum = torch.zeros(lse.shape, device=DEV)
    dq, dk, dv, dw, db = flash_spacetime_backward(q, k, v, feats, w, b, None, lse, do, cu_seqlens=cu, rowsum=rowsum)
    torch.cuda.synchronize()
    for name, t in (("out", out), ("lse", lse), ("dq", dq), ("dk", dk), ("dv", dv), ("rowsum", rowsum),
                    ("dW", dw), ("db", db)):
        assert torch.isnan(t).all(), f"{name} is not NaN everywhere"
    # A well-formed call on the same buffers afterwards is unaffected.
    good = torch.tensor([0, 800, 800, 1600], dtype=torch.int32, device=DEV)
    out2, _ = flash_spacetime_forward(q, k, v, feats, w, b, None, cu_seqlens=good)
    torch.cuda.synchronize()
    assert torch.isfinite(out2).all()
