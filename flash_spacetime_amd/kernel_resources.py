"""Registers, spills and occupancy of the built kernels, as the compiler
reports them for the code objects (kernel-resource-usage remarks recorded by
`flash_spacetime_amd.build` in csrc/_build/kernel_resources.json).

Usage: python -m flash_spacetime_amd.kernel_resources [REGEX ...]
prints a markdown table of the kernel instances whose demangled name matches
any REGEX (all instances without one). A VGPR figure here is the count the
hardware allocates for the kernel, which sets its waves per SIMD; scratch is
the per-lane spill space (0: no spills).
"""

from __future__ import annotations

import json
import re
import subprocess
import sys

from .build import RESOURCES


def demangle(names):
    try:
        res = subprocess.run(["c++filt"], input="\n".join(names), capture_output=True, text=True, check=True)
        return res.stdout.splitlines()
    except (OSError, subprocess.CalledProcessError):
        return list(names)


def table(patterns=()):
    data = json.loads(RESOURCES.read_text())
    names = sorted(data)
    pretty = dict(zip(names, demangle(names)))
    rows = ["| kernel instance | VGPRs | AGPRs | scratch (bytes/lane) | waves / SIMD |", "|---|---|---|---|---|"]
    for n in names:
        p = pretty[n].replace("(fst::FwdParams)", "").replace("(fst::BwdParams)", "").replace("fst::", "")
        if patterns and not any(re.search(pat, p) for pat in patterns):
            continue
        d = data[n]
        rows.append(f"| `{p}` | {d.get('vgpr', '')} | {d.get('agpr', '')} | {d.get('scratch_bytes', '')} | "
                    f"{d.get('waves_per_simd', '')} |")
    return "\n".join(rows)


if __name__ == "__main__":
    print(table(sys.argv[1:]))
