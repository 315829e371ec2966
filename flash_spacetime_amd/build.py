"""Build the gfx950 HIP library `libflash_spacetime.so` in the package directory.

Every kernel instance family is its own translation unit so hipcc runs them
in parallel; the objects are linked into one shared library whose C ABI is
declared in include/flash_spacetime.h. Usage: python -m flash_spacetime_amd.build
"""

from __future__ import annotations

import json
import os
import re
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = CSRC / "_build"
LIB = PKG / "libflash_spacetime.so"

ARCH = os.environ.get("FST_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Packed fp32 VALU forms are kept out of the device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]

DTYPES = {"bf16": "bf16", "f32": "float"}
HEAD_DIMS = (16, 32, 48, 64)


# The bf16 tile rows kernel is built in a unit of its own with the machine
# scheduler's max-ilp strategy (cfg2's rows kernel 0.891 -> 0.873 ms); the
# strategy slowed the cols kernel by up to a third at other shapes and the
# float32 forward by 11 %, so every other unit keeps the default.
ROWS_SCHED = ["-mllvm", "--amdgpu-sched-strategy=max-ilp"]


def source_hash() -> str:
    """First 12 hex digits of the SHA-256 of every kernel source: the build id
    fst_version reports (the tuner's plan cache keys on it)."""
    import hashlib

    h = hashlib.sha256()
    for p in sorted(CSRC.glob("*.h")) + sorted(CSRC.glob("*.hip")):
        h.update(p.name.encode())
        h.update(p.read_bytes())
    return h.hexdigest()[:12]


def _units():
    units = [("capi", CSRC / "fst_capi.hip", [f'-DFST_BUILD_ID="{source_hash()}"'])]
    for tag, ctype in DTYPES.items():
        for d in HEAD_DIMS:
            name = f"{tag}_{d}"
            defs = [f"-DFST_T={ctype}", f"-DFST_D={d}", f"-DFST_NAME={name}"]
            units.append((f"fwd_{name}", CSRC / "fst_fwd_inst.hip", defs))
            if tag == "bf16":
                units.append((f"bwdr_{name}", CSRC / "fst_bwd_inst.hip", defs + ["-DFST_BWD_PART=1"] + ROWS_SCHED))
                units.append((f"bwd_{name}", CSRC / "fst_bwd_inst.hip", defs + ["-DFST_BWD_PART=2"]))
            else:
                units.append((f"bwd_{name}", CSRC / "fst_bwd_inst.hip", defs))
    return [u for u in units if u[1].exists()]


RESOURCES = BUILD / "kernel_resources.json"
_REMARK = re.compile(r"remark:\s+(Function Name|VGPRs|AGPRs|ScratchSize \[bytes/lane\]|Occupancy \[waves/SIMD\]"
                     r"|LDS Size \[bytes/block\]): (\S+)")
_KEYS = {"VGPRs": "vgpr", "AGPRs": "agpr", "ScratchSize [bytes/lane]": "scratch_bytes",
         "Occupancy [waves/SIMD]": "waves_per_simd", "LDS Size [bytes/block]": "static_lds_bytes"}


def _resources(text):
    """Per-kernel register, scratch and occupancy figures from the compiler's
    kernel-resource-usage remarks of one unit (the code object's own counts)."""
    out, cur = {}, None
    for line in text.splitlines():
        m = _REMARK.search(line)
        if not m:
            continue
        key, val = m.group(1), m.group(2)
        if key == "Function Name":
            cur = out.setdefault(val, {})
        elif cur is not None:
            cur[_KEYS[key]] = int(val)
    return out


def _compile(unit):
    name, src, defs = unit
    obj = BUILD / f"{name}.o"
    cmd = [HIPCC, *FLAGS, *defs, "-c", str(src), "-o", str(obj), "-Rpass-analysis=kernel-resource-usage"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    text = res.stdout + res.stderr
    out = "\n".join(
        line for line in text.splitlines()
        if "packed-fp32-ops" not in line and "-Rpass-analysis=kernel-resource-usage" not in line
    )
    return name, obj, res.returncode, out, _resources(text)


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile every unit (always) and link the shared library."""
    BUILD.mkdir(parents=True, exist_ok=True)
    units = _units()
    jobs = jobs or min(len(units), max(1, min(16, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        results = list(pool.map(_compile, units))
    failed = [r for r in results if r[2] != 0]
    for name, _, rc, out, _ in results:
        if out.strip() and (verbose or rc != 0):
            print(f"--- {name} ---\n{out}", file=sys.stderr)
    if failed:
        raise RuntimeError("hipcc failed for: " + ", ".join(r[0] for r in failed))
    resources = {}
    for r in results:
        resources.update(r[4])
    RESOURCES.write_text(json.dumps(resources, indent=0, sort_keys=True))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-o", str(tmp), *(str(r[1]) for r in results)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("link failed:\n" + res.stdout + res.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
