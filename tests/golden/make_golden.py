"""Write golden input/output vectors of the reference specification.

Run once, in the build container only (the reference checkout does not exist
on the GPU box):  python tests/golden/make_golden.py /root/reference

It imports the reference's pure-PyTorch spec module
(`src/flash_spacetime/reference.py`, torch-only, no Triton) on the CPU and
records, for small seeded inputs, what `sinusoidal_frequencies`,
`spacetime_pair_features`, `pair_mask_bias` and
`spacetime_attention_reference` return in float64, float32 and bfloat16.
These pin the parts of the CPU oracle that closed forms cannot: the exact
dtype plumbing of the eager definition (emb cast to the weight dtype, fp32
mask promotion, `p.to(v.dtype)`). The reference requires C == D, so every
case here has C == D; the generalised W [D, C] is pinned by closed forms.

Only the vectors (inputs and outputs, as a .npz of float arrays; bf16 values
are widened exactly to float32) are committed; nothing of the reference is.
"""

import importlib.util
import sys
from pathlib import Path

import numpy as np
import torch


def _load_spec(root: Path):
    path = root / "src" / "flash_spacetime" / "reference.py"
    spec = importlib.util.spec_from_file_location("_fst_reference_spec", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _np(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.bfloat16:
        t = t.float()
    return t.detach().cpu().numpy()


def main() -> None:
    root = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    ref = _load_spec(root)
    out = {}
    for c in (16, 32, 48, 64):
        out[f"freqs_C{c}"] = _np(ref.sinusoidal_frequencies(c, torch.device("cpu")))
    out["time_scale"] = np.array([ref.TIME_SCALE], dtype=np.float64)

    flags_list = [(True, True), (True, False), (False, True), (False, False)]
    cases = [
        # name, B, L, H, D, raw-unit coordinates?
        ("n16", 2, 7, 2, 16, False),
        ("r16", 2, 5, 3, 16, True),
        ("n32", 1, 9, 2, 32, False),
    ]
    for name, bsz, length, heads, dim, raw in cases:
        gen = torch.Generator().manual_seed(1000 + dim + length)
        q = torch.randn(bsz, heads, length, dim, generator=gen, dtype=torch.float64)
        k = torch.randn(bsz, heads, length, dim, generator=gen, dtype=torch.float64)
        v = torch.randn(bsz, heads, length, dim, generator=gen, dtype=torch.float64)
        if raw:
            xyz = (torch.rand(bsz, length, 3, generator=gen, dtype=torch.float64) - 0.5) * 1000
            t = torch.rand(bsz, length, 1, generator=gen, dtype=torch.float64) * 2e4
            feats = torch.cat([xyz, t, torch.randn(bsz, length, 1, generator=gen, dtype=torch.float64)], -1)
        else:
            feats = torch.randn(bsz, length, 5, generator=gen, dtype=torch.float64)
        # one light-like pair (I == 0 exactly) in event 0: tokens 0 and 1
        feats[0, 1, :4] = feats[0, 0, :4] + torch.tensor([18.0, 0.0, 0.0, 1.0], dtype=torch.float64)
        weight = torch.randn(dim, dim, generator=gen, dtype=torch.float64) / dim ** 0.5
        bias = torch.randn(dim, generator=gen, dtype=torch.float64)
        seqlens = torch.tensor([length] + [max(1, length - 3)] * (bsz - 1), dtype=torch.long)
        valid = ref.valid_row_mask(bsz, length, seqlens)
        mask = ref.float_padding_mask(valid, torch.float32)
        for key, val in dict(q=q, k=k, v=v, feats=feats, weight=weight, bias=bias).items():
            out[f"{name}_{key}"] = _np(val)
        out[f"{name}_seqlens"] = seqlens.numpy()
        out[f"{name}_pairmask"] = _np(ref.pair_mask_bias(mask))
        for dt, tag in ((torch.float64, "f64"), (torch.float32, "f32"), (torch.bfloat16, "bf16")):
            fdt = torch.float64 if dt == torch.float64 else torch.float32
            rel = ref.spacetime_pair_features(feats.to(fdt), weight.to(dt), bias.to(dt))
            out[f"{name}_rel_{tag}"] = _np(rel)
            for fl in flags_list:
                o = ref.spacetime_attention_reference(
                    q.to(dt), k.to(dt), v.to(dt), feats.to(fdt), weight.to(dt), bias.to(dt),
                    key_padding_mask=mask, use_attn_bias=fl[0], use_activation_bias=fl[1],
                )
                out[f"{name}_out_{tag}_{int(fl[0])}{int(fl[1])}"] = _np(o)
    dest = Path(__file__).with_name("reference_spec_vectors.npz")
    np.savez_compressed(dest, **out)
    print(f"wrote {dest} ({dest.stat().st_size} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
