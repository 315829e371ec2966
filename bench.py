"""Benchmark of the fused spacetime-bias attention step on one MI355X.

Workload (the metric's configuration): one
forward + backward of `flash_spacetime_attention` at B=256, L=768, H=12,
D=32, C=16 in bf16 with per-event valid lengths ~ U{16..768}. Inputs are
synthetic and drawn from one seeded CPU generator in a fixed order
(q, k, v, pos, W, b, lengths, dO): q, k, v, dO ~ N(0, 1); x, y, z ~
U(-500, 500), t ~ U(0, 2e4); W ~ N(0, 1/C) and b ~ N(0, 0.02) in fp32.

Prints ONE JSON line: ms/step of the whole fwd+bwd step (HIP events over K
steps after W warm-up steps, inputs resident in HBM), peak GiB allocated
by the step, % of the bf16 MFMA peak for the algorithmic FLOPs, per-kernel
times of the individual launches, the MFMA roofline of the dominant kernel,
and the CPU baseline (the oracle's eager restatement of the spec, fp32,
fwd+bwd, timed on this host's cores on a bounded sample of events).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--autotune]
       [--workload cfg2|cfg1|cfg3|cfg4|cfg4-fp32|cfg2-model|lscale|plans]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import torch  # noqa: E402

METRIC = "fwd+bwd ms/step & peak GiB at B=256,L=768,C=16 bf16; % MFMA peak"
B, L, H, D, C = 256, 768, 12, 32, 16
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0


# Position distribution of the synthetic inputs (--pos): "detector" draws the
# BASELINE configs' x, y, z ~ U(-500, 500), t ~ U(0, 2e4) (every off-diagonal
# pair saturates the angle clip, so E is nearly constant), "normal" the
# survey's twin with pos ~ N(0, 1) [.., 4], which exercises E for real.
POS = "detector"


def draw_pos(gen, *lead):
    """Positions [*lead, 4] from `gen` in the distribution POS names."""
    if POS == "normal":
        return torch.randn(*lead, 4, generator=gen)
    xyz = (torch.rand(*lead, 3, generator=gen) - 0.5) * 1000.0
    t = torch.rand(*lead, 1, generator=gen) * 2e4
    return torch.cat([xyz, t], -1)


def make_inputs(device):
    gen = torch.Generator().manual_seed(0)
    q = torch.randn(B, H, L, D, generator=gen)
    k = torch.randn(B, H, L, D, generator=gen)
    v = torch.randn(B, H, L, D, generator=gen)
    feats = draw_pos(gen, B, L)
    w = torch.randn(D, C, generator=gen) / C ** 0.5
    bias = torch.randn(D, generator=gen) * 0.02
    lengths = torch.randint(16, L + 1, (B,), generator=gen)
    do = torch.randn(B, H, L, D, generator=gen)
    pad_mask = torch.arange(L)[None, :] >= lengths[:, None]  # bool key_padding_mask, True = padding
    return dict(
        q=q.to(device, torch.bfloat16), k=k.to(device, torch.bfloat16), v=v.to(device, torch.bfloat16),
        feats=feats.to(device), w=w.to(device), b=bias.to(device), lengths=lengths,
        pad_mask=pad_mask.to(device), do=do.to(device, torch.bfloat16),
    )


def flop_counts(lengths):
    """Algorithmic FLOPs over valid pairs (per pair-head): fwd 4(D+C);
    bwd 10D+8C, of which the rows kernel is credited 6D+8C (one S and dP
    recompute, dq, H, G) and the cols kernel 4D (dk, dv)."""
    sl2 = float((lengths.double() ** 2).sum())
    return {
        "fwd": H * sl2 * 4 * (D + C),
        "bwd_rows": H * sl2 * (6 * D + 8 * C),
        "bwd_cols": H * sl2 * 4 * D,
        "sum_l2": sl2,
        "dense_fwd_bwd": H * B * L * L * (4 * (D + C) + 10 * D + 8 * C),
    }


def time_events(fn, iters, stream):
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(iters):
        fn()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / iters


def current_plan():
    """FST_PLAN_* bits the operators ran with: the tuner's choices (one forward
    and one backward entry per workload), 0 for the library's static plan."""
    from flash_spacetime_amd import tune

    plan = 0
    for bits in tune.chosen().values():
        plan |= bits
    return plan


def plan_label(plan):
    from flash_spacetime_amd import tune

    return tune.plan_names(plan) if plan else "static"


def kernel_times(inp, seqlens, iters=10, cu=None, plan=0, flags=(True, True), with_out=True):
    """Average duration of each launch, timed with HIP events on the stream the
    library launches on (torch's current stream), one phase at a time, with
    the FST_PLAN_* bits `plan` (0: the library's static choice). with_out:
    the backward is given the forward's output, as the autograd op gives it
    (its rows kernel's reference D); else it forms D online."""
    from flash_spacetime_amd import _lib
    from flash_spacetime_amd.forward import _Prepared

    lib = _lib.load()
    dev = inp["q"].device
    prep = _Prepared(inp["q"], inp["k"], inp["v"], inp["feats"], inp["w"], inp["b"], seqlens, None,
                     flags[0], flags[1], cu)
    d_, c_ = inp["w"].shape
    dims = prep.dims()
    dims = (dims[0], dims[1] | plan) + tuple(dims[2:])
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream
    out = torch.empty_like(prep.q)
    lse = torch.empty(prep.vec_shape(), device=dev, dtype=torch.float32)
    fws = lib.fst_forward_workspace_bytes(*dims)
    fwork = torch.empty(fws, device=dev, dtype=torch.uint8)
    P = _lib.ptr
    fargs = (P(prep.q), P(prep.k), P(prep.v), P(prep.pos4), P(prep.weight), P(prep.bias), P(prep.lens),
             prep.scale, P(out), P(lse), P(fwork), fws, sh)
    _lib.check(lib.fst_forward_phases(_lib.FST_PHASE_WORKLIST, *dims, *fargs), "worklist")
    do = inp["do"].contiguous()
    dq, dk, dv = (torch.empty_like(prep.q) for _ in range(3))
    dw = torch.empty(d_, c_, device=dev)
    db = torch.empty(d_, device=dev)
    bws = lib.fst_backward_workspace_bytes(*dims)
    bwork = torch.empty(bws, device=dev, dtype=torch.uint8)
    bargs = (P(prep.q), P(prep.k), P(prep.v), P(prep.pos4), P(prep.weight), P(prep.bias), P(prep.lens), P(lse),
             P(do), P(out) if with_out else None, prep.scale, P(dq), P(dk), P(dv), P(dw), P(db), None, P(bwork),
             bws, sh)
    _lib.check(lib.fst_forward_phases(_lib.FST_PHASE_FWD, *dims, *fargs), "fwd")
    _lib.check(lib.fst_backward_phases(_lib.FST_BWD_ALL, *dims, *bargs), "bwd")
    torch.cuda.synchronize(dev)
    res = {}
    res["fwd"] = time_events(lambda: lib.fst_forward_phases(_lib.FST_PHASE_FWD, *dims, *fargs), iters, stream)
    res["bwd_rows"] = time_events(lambda: lib.fst_backward_phases(_lib.FST_PHASE_BWD_ROWS, *dims, *bargs), iters,
                                  stream)
    res["bwd_cols"] = time_events(lambda: lib.fst_backward_phases(_lib.FST_PHASE_BWD_COLS, *dims, *bargs), iters,
                                  stream)
    res["bwd_reduce"] = time_events(lambda: lib.fst_backward_phases(_lib.FST_PHASE_REDUCE, *dims, *bargs), iters,
                                    stream)
    res["worklist"] = time_events(lambda: lib.fst_forward_phases(_lib.FST_PHASE_WORKLIST, *dims, *fargs), iters,
                                  stream)
    return res


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_cfg2.json")


def measured_traffic(phase):
    """HBM bytes per launch of `phase` from the committed rocprofv3 counter
    summary (FETCH_SIZE + WRITE_SIZE, calibrated against a copy of known size;
    written by flash_spacetime_amd.rocprof_summary), or None when absent."""
    try:
        with open(TRAFFIC_FILE) as f:
            entry = json.load(f)["kernels"].get(phase)
    except (OSError, ValueError, KeyError):
        return None
    return None if entry is None else round(float(entry["bytes"]))


def calibration_copy(dev, nbytes=2 ** 30):
    """fp32 multiply by 1.0 over `nbytes`: one read and one write per element."""
    src = torch.ones(nbytes // 4, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize(dev)
    del src, dst


def cpu_model():
    """The host CPU as /proc/cpuinfo names it: model name, family / model /
    stepping numbers (virtual machines often report a generic name) and the
    logical CPUs this process may use; else the platform string."""
    fields = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                key, _, val = line.partition(":")
                key = key.strip()
                if key in ("model name", "cpu family", "model", "stepping") and key not in fields:
                    fields[key] = val.strip()
                if not line.strip() and fields:
                    break
    except OSError:
        pass
    if "model name" not in fields:
        import platform

        return platform.processor() or platform.machine()
    ids = ", ".join(f"{k} {fields[k]}" for k in ("cpu family", "model", "stepping") if k in fields)
    return f"{fields['model name']} ({ids}; {len(os.sched_getaffinity(0))} logical CPUs available)"


def _cpu_eager_ms(inp, dtype, budget_s, max_events):
    """Per-event ms of the oracle's eager fwd+bwd in `dtype` on the CPU,
    one padded event at a time until the budget is spent; (ms, events)."""
    import oracle

    q = inp["q"].to(dtype).cpu()
    k = inp["k"].to(dtype).cpu()
    v = inp["v"].to(dtype).cpu()
    feats = inp["feats"].float().cpu()
    w, b = inp["w"].to(dtype).cpu(), inp["b"].to(dtype).cpu()
    do = inp["do"].to(dtype).cpu()
    valid = ~inp["pad_mask"].cpu()
    fmask = oracle.float_padding_mask(valid, torch.float32)
    done, t_total = 0, 0.0
    while done < max_events and (t_total < budget_s or done == 0):
        sl = slice(done, done + 1)
        leaves = [x[sl].clone().requires_grad_(True) for x in (q, k, v)]
        wl, bl = w.clone().requires_grad_(True), b.clone().requires_grad_(True)
        t0 = time.perf_counter()
        out = oracle.attention(*leaves, feats[sl], wl, bl, key_padding_mask=fmask[sl])
        out.backward(do[sl] * valid[sl][:, None, :, None].to(dtype))
        t_total += time.perf_counter() - t0
        done += 1
    return 1e3 * t_total / done, done, t_total


def cpu_baseline(inp, budget_s=15.0, max_events=B, bf16_budget_s=5.0):
    """The oracle's eager restatement of the spec (materialised R, autograd
    backward) on this host's CPU cores: fp32 (`value`) and bf16, padded
    events of length L with the float mask exactly as the eager module runs,
    timed one event at a time until each time budget is spent; ms/step is
    extrapolated to the 256 events (eager padded cost is the same for every
    event)."""
    torch.set_num_threads(os.cpu_count() or 1)
    threads = torch.get_num_threads()
    ms32, n32, t32 = _cpu_eager_ms(inp, torch.float32, budget_s, max_events)
    ms16, n16, t16 = _cpu_eager_ms(inp, torch.bfloat16, bf16_budget_s, max_events)
    return {
        "value": ms32 * B,
        "unit": "ms",
        "cores": threads,
        "cpu_model": cpu_model(),
        "kind": "port",
        "sample": f"{n32} of {B} padded events (L={L}) fwd+bwd in fp32 eager PyTorch on the CPU "
                  f"(oracle.attention + autograd, materialised [1,L,L,D] pair tensor), {1e3 * t32:.0f} ms "
                  f"total, extrapolated x{B}/{n32}",
        "bf16_value": ms16 * B,
        "bf16_sample": f"{n16} of {B} events in bf16 (same restatement, bf16 operands), {1e3 * t16:.0f} ms total, "
                       f"extrapolated x{B}/{n16}",
    }


WORKLOADS = {
    "cfg3": "configs[3]: flash_spacetime_attention_varlen fwd+bwd, 4096 packed events, lengths "
            "round(lognormal(5, 1)) in [1, 3000] with 1% of length 1, H=12 D=32 C=16 bf16",
    "cfg4": "configs[4]: flash_spacetime_attention fwd+bwd, B=8 L=4096 (no padding) H=8 D=64 C=64, "
            "q and k x30, bf16",
    "cfg4-fp32": "configs[4]: flash_spacetime_attention fwd+bwd, B=8 L=4096 (no padding) H=8 D=64 C=64, "
                 "q and k x30, fp32",
    "cfg1": "configs[1]: flash_spacetime_attention forward only, B=256 L=768 H=12 D=32 C=16 bf16, valid "
            "lengths U{16..768} (bool key_padding_mask -> seqlens once), W/b fp32",
    "lscale": "configs[2] at L = 384, 768, 1536: flash_spacetime_attention fwd+bwd, B=256 H=12 D=32 C=16 "
              "bf16, lengths U{16..L}",
    "plans": "per-kernel times of every supported FST_PLAN_* combination of each kernel family against the "
             "static choice: bf16 cfg2, cfg3, cfg4 and seven other head layouts, fp32 cfg4, cfg2 and one small",
    "cfg2-model": "SpacetimeAttention fwd+bwd (fused QKV linear, flash_spacetime_attention_qkv, output "
                  "linear) at cfg2 sizes: x [256, 768, 384] bf16, H=12 D=32 C=16, lengths U{16..768}",
}


def run_forward_only(steps, warmup):
    """the forward alone at cfg2's shape (the op under no_grad, the
    bool key_padding_mask converted to lengths once): ms/step, peak GiB above
    the inputs, and the MFMA fraction of the forward's algorithmic FLOPs."""
    from flash_spacetime_amd import flash_spacetime_attention
    from flash_spacetime_amd.forward import lengths_from_mask

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    inp = make_inputs(dev)
    seqlens = lengths_from_mask(inp["pad_mask"], L)

    def step():
        with torch.no_grad():
            flash_spacetime_attention(inp["q"], inp["k"], inp["v"], inp["feats"], inp["w"], inp["b"], seqlens)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize(dev)
    ms = time_events(step, steps, torch.cuda.current_stream(dev))
    torch.cuda.synchronize(dev)
    torch.cuda.reset_peak_memory_stats(dev)
    base = torch.cuda.memory_allocated(dev)
    step()
    torch.cuda.synchronize(dev)
    peak = (torch.cuda.max_memory_allocated(dev) - base) / 2 ** 30
    f_fwd = flop_counts(inp["lengths"])["fwd"]
    print(json.dumps({
        "metric": "fwd ms/step & peak GiB at B=256,L=768,C=16 bf16; % MFMA peak", "value": round(ms, 4),
        "unit": "ms", "n_gpus": 1, "steps": steps, "warmup": warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded; BASELINE.json configs[1] distributions)",
        "config": {"workload": WORKLOADS["cfg1"], "positions": POS}, "peak_gib": round(peak, 4),
        "mfma_pct_of_peak": round(100.0 * f_fwd / (ms * 1e-3) / (PEAK_BF16_TFLOPS * 1e12), 3),
    }), flush=True)


def run_length_scaling(steps, warmup):
    """cfg2's step at L = 384, 768, 1536 (B = 256, lengths U{16..L}, same
    distributions): ms/step, peak GiB above the inputs, valid pairs. Time
    follows the valid pairs (sum of squared lengths); memory grows linearly
    in L (nothing O(L^2) is materialised)."""
    from flash_spacetime_amd import flash_spacetime_attention

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    out = {}
    for length in (384, 768, 1536):
        gen = torch.Generator().manual_seed(length)
        rn = lambda *s_: torch.randn(*s_, generator=gen)
        q, k, v, do = (rn(B, H, length, D).to(dev, torch.bfloat16) for _ in range(4))
        feats = torch.cat([(torch.rand(B, length, 3, generator=gen) - 0.5) * 1000.0,
                           torch.rand(B, length, 1, generator=gen) * 2e4], -1).to(dev)
        w = (rn(D, C) / C ** 0.5).to(dev)
        bias = (rn(D) * 0.02).to(dev)
        lens = torch.randint(16, length + 1, (B,), generator=gen)
        seqlens = lens.to(dev, torch.int32)
        leaves = [x.clone().requires_grad_(True) for x in (q, k, v)]
        wl, bl = w.clone().requires_grad_(True), bias.clone().requires_grad_(True)

        def step():
            for t_ in (*leaves, wl, bl):
                t_.grad = None
            flash_spacetime_attention(*leaves, feats, wl, bl, seqlens).backward(do)

        for _ in range(warmup):
            step()
        torch.cuda.synchronize(dev)
        ms = time_events(step, steps, torch.cuda.current_stream(dev))
        torch.cuda.synchronize(dev)
        for t_ in (*leaves, wl, bl):
            t_.grad = None
        torch.cuda.synchronize(dev)
        torch.cuda.reset_peak_memory_stats(dev)
        base = torch.cuda.memory_allocated(dev)
        step()
        torch.cuda.synchronize(dev)
        peak = (torch.cuda.max_memory_allocated(dev) - base) / 2 ** 30
        out[str(length)] = {"ms": round(ms, 4), "peak_gib": round(peak, 4),
                            "valid_pairs": float((lens.double() ** 2).sum())}
        del q, k, v, do, feats, leaves
        torch.cuda.empty_cache()
    print(json.dumps({
        "metric": "fwd+bwd ms/step and peak GiB vs L at cfg2's other sizes", "value": out["768"]["ms"],
        "unit": "ms", "n_gpus": 1, "steps": steps, "warmup": warmup, "ms_per_step": out["768"]["ms"],
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded; cfg2 distributions at each L)",
        "config": {"workload": WORKLOADS["lscale"]}, "by_length": out,
    }), flush=True)


def run_model_workload(steps, warmup):
    """The model-side caller at cfg2 sizes: one fwd+bwd of `SpacetimeAttention`
    (x -> fused QKV GEMM -> fused op on the interleaved projection -> output
    GEMM, gradients of x and every parameter). Beside it, the same module's
    parameters run the way the reference's caller runs them: three linears,
    split heads made contiguous, the op, heads merged by a copy, output
    linear (`split_heads_copies_ms`)."""
    from flash_spacetime_amd import SpacetimeAttention, flash_spacetime_attention, merge_heads

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    inp = make_inputs(dev)
    from flash_spacetime_amd.forward import lengths_from_mask

    seqlens = lengths_from_mask(inp["pad_mask"], L)
    dim = H * D
    torch.manual_seed(5)
    mod = SpacetimeAttention(dim, H, C, qkv_bias=True, device=dev, dtype=torch.bfloat16)
    gen = torch.Generator().manual_seed(6)
    x = torch.randn(B, L, dim, generator=gen).to(dev, torch.bfloat16).requires_grad_(True)
    gy = torch.randn(B, L, dim, generator=gen).to(dev, torch.bfloat16)
    feats = inp["feats"]
    params = [x, *mod.parameters()]

    def fused():
        for t_ in params:
            t_.grad = None
        mod(x, feats, seqlens).backward(gy)

    def reference_caller():
        for t_ in params:
            t_.grad = None
        q = torch.nn.functional.linear(x, mod.proj_q.weight, mod.q_bias)
        k = torch.nn.functional.linear(x, mod.proj_k.weight)
        v = torch.nn.functional.linear(x, mod.proj_v.weight, mod.v_bias)
        heads = [t_.view(B, L, H, D).transpose(1, 2).contiguous() for t_ in (q, k, v)]
        o = flash_spacetime_attention(*heads, feats, mod.rel_proj.weight, mod.rel_proj.bias, seqlens)
        mod.proj(merge_heads(o).contiguous()).backward(gy)

    stream = torch.cuda.current_stream(dev)
    res = {}
    for name, fn in (("fused", fused), ("reference_caller", reference_caller)):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize(dev)
        res[name] = time_events(fn, steps, stream)
        torch.cuda.synchronize(dev)
    print(json.dumps({
        "metric": "SpacetimeAttention fwd+bwd ms/step at cfg2 sizes", "value": round(res["fused"], 4),
        "unit": "ms", "n_gpus": 1, "steps": steps, "warmup": warmup, "ms_per_step": round(res["fused"], 4),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded; cfg2 lengths and features, random-init module)",
        "config": {"workload": WORKLOADS["cfg2-model"]},
        "split_heads_copies_ms": round(res["reference_caller"], 4),
    }), flush=True)


def run_other_workload(name, steps, warmup):
    """One JSON line for a non-headline BASELINE configuration: ms/step of the
    fwd+bwd step through the operators, per-kernel times and the MFMA fraction
    of the algorithmic FLOPs (fp32 runs are priced at the fp32 matrix peak)."""
    from flash_spacetime_amd import flash_spacetime_attention, flash_spacetime_attention_varlen

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    gen = torch.Generator().manual_seed(3 if name == "cfg3" else 4)
    rn = lambda *s_: torch.randn(*s_, generator=gen)
    if name == "cfg3":
        import math
        h, d, c, n_ev = 12, 32, 16, 4096
        lens = torch.exp(5.0 + torch.randn(n_ev, generator=gen, dtype=torch.float64)).round().clamp(1, 3000).long()
        lens[torch.randperm(n_ev, generator=gen)[: math.ceil(0.01 * n_ev)]] = 1
        total = int(lens.sum())
        dtype = torch.bfloat16
        shape = (total, h, d)
        pos = draw_pos(gen, total)
        cu = torch.zeros(n_ev + 1, dtype=torch.int32)
        cu[1:] = torch.cumsum(lens, 0)
        cu = cu.to(dev)
        scale_qk = 1.0
    else:
        h, d, c, bsz, length = 8, 64, 64, 8, 4096
        lens = torch.full((bsz,), length, dtype=torch.long)
        dtype = torch.float32 if name == "cfg4-fp32" else torch.bfloat16
        shape = (bsz, h, length, d)
        pos = draw_pos(gen, bsz, length)
        cu = None
        scale_qk = 30.0
    q = (rn(*shape) * scale_qk).to(dev, dtype)
    k = (rn(*shape) * scale_qk).to(dev, dtype)
    v = rn(*shape).to(dev, dtype)
    feats = pos.to(dev)
    w = (rn(d, c) / c ** 0.5).to(dev)
    bias = (rn(d) * 0.02).to(dev)
    do = rn(*shape).to(dev, dtype)
    seqlens = None if cu is not None else lens.to(dev, torch.int32)
    leaves = [x.detach().clone().requires_grad_(True) for x in (q, k, v)]
    wl, bl = w.clone().requires_grad_(True), bias.clone().requires_grad_(True)

    def step():
        for t_ in (*leaves, wl, bl):
            t_.grad = None
        if cu is not None:
            out = flash_spacetime_attention_varlen(*leaves, feats, wl, bl, cu)
        else:
            out = flash_spacetime_attention(*leaves, feats, wl, bl, seqlens)
        out.backward(do)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize(dev)
    stream = torch.cuda.current_stream(dev)
    ms = time_events(step, steps, stream)
    torch.cuda.synchronize(dev)
    inp = dict(q=q, k=k, v=v, feats=feats, w=w, b=bias, do=do)
    plan = current_plan()
    kt = kernel_times(inp, seqlens, cu=cu, plan=plan)
    sl2 = float((lens.double() ** 2).sum())
    f_total = h * sl2 * (4 * (d + c) + 10 * d + 8 * c)
    peak = PEAK_BF16_TFLOPS if dtype == torch.bfloat16 else 157.3
    print(json.dumps({
        "metric": f"fwd+bwd ms/step at {name}", "value": round(ms, 4), "unit": "ms", "n_gpus": 1,
        "steps": steps, "warmup": warmup, "ms_per_step": round(ms, 4), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16" if dtype == torch.bfloat16 else "fp32",
        "data": "synthetic (seeded; BASELINE.json distributions)",
        "config": {"workload": WORKLOADS[name], "valid_pairs": sl2, "positions": POS},
        "plan": plan_label(plan),
        "mfma_pct_of_peak": round(100.0 * f_total / (ms * 1e-3) / (peak * 1e12), 3),
        "algorithmic_tflop": round(f_total / 1e12, 4),
        "kernels_ms": {k_: round(v_, 4) for k_, v_ in kt.items()},
    }), flush=True)


PLAN_SHAPES = [
    # (name, dtype, H, D, C, B, L (None: cfg3's packed events), full-length events, (attn, act bias))
    ("cfg2", "bf16", 12, 32, 16, 256, 768, False, (True, True)),
    ("cfg2, use_activation_bias=False", "bf16", 12, 32, 16, 256, 768, False, (True, False)),
    ("cfg3", "bf16", 12, 32, 16, 4096, None, False, (True, True)),
    ("cfg4", "bf16", 8, 64, 64, 8, 4096, True, (True, True)),
    ("H=8 D=32 C=16", "bf16", 8, 32, 16, 128, 1024, False, (True, True)),
    ("H=16 D=16 C=16", "bf16", 16, 16, 16, 128, 1024, False, (True, True)),
    ("H=4 D=64 C=16", "bf16", 4, 64, 16, 256, 512, False, (True, True)),
    ("H=12 D=16 C=32", "bf16", 12, 16, 32, 128, 768, False, (True, True)),
    ("H=8 D=48 C=16", "bf16", 8, 48, 16, 128, 768, False, (True, True)),
    ("H=12 D=64 C=32", "bf16", 12, 64, 32, 64, 1024, False, (True, True)),
    ("cfg4-fp32", "fp32", 8, 64, 64, 8, 4096, True, (True, True)),
    ("cfg2-fp32", "fp32", 12, 32, 16, 256, 768, False, (True, True)),
    ("H=4 D=16 C=16 fp32", "fp32", 4, 16, 16, 128, 1024, False, (True, True)),
]


def run_plan_sweep(steps, warmup):
    """Per-kernel times (ms) of every compiled variant (FST_PLAN_*) of the
    forward, rows and cols kernels, and of the library's static choice: for
    each kernel family, every supported combination of its plan groups (one
    offered bit per group), over bf16 and fp32 shapes with lengths U{16..L}
    (cfg3: its packed lognormal events; cfg4: full-length events)."""
    import math

    from flash_spacetime_amd import _lib, tune

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    gen = torch.Generator().manual_seed(11)
    rows_out = []
    for name, dt, h, d, c, bsz, length, full, flags in PLAN_SHAPES:
        rn = lambda *s_: torch.randn(*s_, generator=gen)  # noqa: E731
        tdt = torch.bfloat16 if dt == "bf16" else torch.float32
        if length is None:
            lens = torch.exp(5.0 + torch.randn(bsz, generator=gen, dtype=torch.float64)).round().clamp(1, 3000).long()
            lens[torch.randperm(bsz, generator=gen)[: math.ceil(0.01 * bsz)]] = 1
            total = int(lens.sum())
            shape, fshape = (total, h, d), (total,)
            cu = torch.zeros(bsz + 1, dtype=torch.int32)
            cu[1:] = torch.cumsum(lens, 0)
            cu, seqlens = cu.to(dev), None
        else:
            lens = torch.full((bsz,), length) if full else torch.randint(16, length + 1, (bsz,), generator=gen)
            shape, fshape = (bsz, h, length, d), (bsz, length)
            cu, seqlens = None, lens.to(dev, torch.int32)
        inp = {n_: rn(*shape).to(dev, tdt) for n_ in ("q", "k", "v", "do")}
        inp["feats"] = torch.cat([(torch.rand(*fshape, 3, generator=gen) - 0.5) * 1000.0,
                                  torch.rand(*fshape, 1, generator=gen) * 2e4], -1).to(dev)
        inp["w"] = (rn(d, c) / c ** 0.5).to(dev)
        inp["b"] = (rn(d) * 0.02).to(dev)
        dtype = _lib.FST_BF16 if dt == "bf16" else _lib.FST_F32
        dims = (dtype, 3, bsz, h, length or 0, int(lens.sum()), d, c)
        families = {"fwd": (tune._combos(dims, tune._FWD_GROUPS), ("fwd",)),
                    "bwd_rows": (tune._combos(dims, tune._ROWS_GROUPS), ("bwd_rows",)),
                    "bwd_cols": (tune._combos(dims, tune._COLS_GROUPS), ("bwd_cols",)),
                    "bwd_fp32": (tune._combos(dims, tune._BWD_GROUPS), ("bwd_rows", "bwd_cols"))}
        res = {}
        iters = max(steps // 4, 3) if full else max(steps // 2, 5)
        for _ in range(2):  # two interleaved rounds; the minimum of each is kept
            for fam, (combos, kernels) in families.items():
                if not combos:
                    continue
                for plan in [0, *combos]:
                    kt = kernel_times(inp, seqlens, iters=iters, cu=cu, plan=plan, flags=flags)
                    label = tune.plan_names(plan) or "static"
                    t_ = sum(kt[k_] for k_ in kernels)
                    res.setdefault(fam, {})[label] = min(res.get(fam, {}).get(label, float("inf")), t_)
        rows_out.append({"shape": name, "dtype": dt, "plans": tune.plan_names(tune.plans(dtype, h, d, c)),
                         **{k_: {l_: round(t_, 4) for l_, t_ in v_.items()} for k_, v_ in res.items()}})
        print(json.dumps(rows_out[-1]), flush=True)
        del inp
        torch.cuda.empty_cache()
    print(json.dumps({
        "metric": "per-kernel ms of each compiled plan variant", "unit": "ms", "n_gpus": 1, "dtype": "bf16+fp32",
        "higher_is_better": False, "data": "synthetic (seeded)",
        "config": {"workload": WORKLOADS["plans"]}, "by_shape": rows_out,
    }), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget-s", type=float, default=15.0)
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="after the bench, run a known-size fp32 copy kernel (1 GiB read + 1 GiB written) "
                         "that rocprof counter runs use to scale FETCH_SIZE / WRITE_SIZE")
    ap.add_argument("--workload", default="cfg2", choices=["cfg2", *WORKLOADS],
                    help="cfg2 (default) is the metric's configuration; the others print a line of their own")
    ap.add_argument("--pos", choices=["detector", "normal"], default="detector",
                    help="positions as the BASELINE configs draw them (detector units), or the N(0, 1) twin "
                         "that exercises the pair embedding")
    ap.add_argument("--autotune", action="store_true",
                    help="time the compiled kernel variants of each shape on its first call (a warm-up "
                         "step) and run the fastest; without it the library's static choice runs")
    args = ap.parse_args()
    global POS
    POS = args.pos
    if args.autotune:
        from flash_spacetime_amd import tune

        tune.set_autotune(True)
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build's hot path is single-device (events are independent; "
              f"multi-GPU would shard events with no exchange). --gpus {args.gpus} is not run.", file=sys.stderr)
        sys.exit(2)

    if args.workload == "cfg2-model":
        run_model_workload(args.steps, args.warmup)
        return
    if args.workload == "plans":
        run_plan_sweep(args.steps, args.warmup)
        return
    if args.workload == "cfg1":
        run_forward_only(args.steps, args.warmup)
        return
    if args.workload == "lscale":
        run_length_scaling(args.steps, args.warmup)
        return
    if args.workload != "cfg2":
        run_other_workload(args.workload, args.steps, args.warmup)
        return

    from flash_spacetime_amd import flash_spacetime_attention
    from flash_spacetime_amd.forward import lengths_from_mask

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    inp = make_inputs(dev)
    seqlens = lengths_from_mask(inp["pad_mask"], L)  # the bool mask, converted once (one readback)
    leaves = [inp[n].detach().clone().requires_grad_(True) for n in ("q", "k", "v")]
    wl = inp["w"].clone().requires_grad_(True)
    bl = inp["b"].clone().requires_grad_(True)
    do = inp["do"]

    def step():
        for t in (*leaves, wl, bl):
            t.grad = None
        out = flash_spacetime_attention(*leaves, inp["feats"], wl, bl, seqlens)
        out.backward(do)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize(dev)
    stream = torch.cuda.current_stream(dev)
    ms = time_events(step, args.steps, stream)
    torch.cuda.synchronize(dev)

    # The step's footprint above the resident inputs: the previous step's
    # gradients are released before the baseline is read, so the gradients
    # this step allocates count in the peak.
    for t in (*leaves, wl, bl):
        t.grad = None
    torch.cuda.synchronize(dev)
    torch.cuda.reset_peak_memory_stats(dev)
    base = torch.cuda.memory_allocated(dev)
    step()
    torch.cuda.synchronize(dev)
    peak_gib = (torch.cuda.max_memory_allocated(dev) - base) / 2 ** 30

    flops = flop_counts(inp["lengths"])
    plan = current_plan()
    kt = kernel_times(inp, seqlens, plan=plan)
    f_total = flops["fwd"] + flops["bwd_rows"] + flops["bwd_cols"]
    mfma_pct = 100.0 * f_total / (ms * 1e-3) / (PEAK_BF16_TFLOPS * 1e12)
    dominant = max(("fwd", "bwd_rows", "bwd_cols"), key=lambda k_: kt[k_])
    achieved = flops[dominant] / (kt[dominant] * 1e-3) / 1e12
    traffic = measured_traffic(dominant)
    result = {
        "metric": METRIC,
        "value": round(ms, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded; BASELINE.json configs[2] distributions)" if POS == "detector" else
                "synthetic (seeded; configs[2] with positions ~ N(0, 1))",
        "config": {
            "workload": "configs[2]: flash_spacetime_attention fwd+bwd, B=256 L=768 H=12 D=32 C=16 bf16, "
                        "valid lengths U{16..768} (bool key_padding_mask -> seqlens once), W/b fp32",
            "B": B, "L": L, "H": H, "D": D, "C": C,
            "valid_pairs": flops["sum_l2"], "positions": POS,
        },
        "plan": plan_label(plan),
        "peak_gib": round(peak_gib, 4),
        "mfma_pct_of_peak": round(mfma_pct, 3),
        "algorithmic_tflop": round(f_total / 1e12, 4),
        "achieved_tflops": round(f_total / (ms * 1e-3) / 1e12, 3),
        "kernels_ms": {k_: round(v_, 4) for k_, v_ in kt.items()},
        "roofline": {
            "kernel": dominant,
            "bound": "mfma",
            "achieved": round(achieved, 3),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 5),
            "traffic": traffic,
            # HBM bytes per launch (rocprofv3 FETCH_SIZE + WRITE_SIZE, calibrated)
            # over this run's launch duration, against the 8 TB/s peak.
            "hbm_gbs": None if traffic is None else round(traffic / (kt[dominant] * 1e-3) / 1e9, 1),
            "hbm_frac": None if traffic is None else round(traffic / (kt[dominant] * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
        },
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(inp, budget_s=args.cpu_budget_s)
    print(json.dumps(result), flush=True)
    if args.calibrate_copy:
        calibration_copy(dev)


if __name__ == "__main__":
    main()
