"""Builds liblongctx100m_attn.so (the C-ABI library) with hipcc for gfx950.

    python -m longctx100m_amd.build [--jobs N]

Every translation unit under csrc/ is compiled to an object in _build/ and
linked into lib/liblongctx100m_attn.so, in-tree, so the library travels with
the source tree.  All HIP code is compiled with packed-fp32 instructions
disabled.  The compiler's per-kernel resource report (registers, scratch,
occupancy, LDS) is written to _build/resource_usage.txt, and the build fails
when a hot kernel uses more scratch memory per lane than SCRATCH_LIMITS
allows (a register array indexed at run time, or a spill inside a hot loop,
costs far more than any tuning gains).
"""

from __future__ import annotations

import argparse
import os
import re
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB_DIR = PKG / "lib"
LIB = LIB_DIR / "liblongctx100m_attn.so"
ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{PKG.parent / 'include'}",
]


# Per-source extras.  layer.hip restates the reference's separately rounded
# tensor ops, and gemv.hip folds the same ops into the decode projections, so
# nothing in either may be contracted into fused multiply-adds.
EXTRA_FLAGS = {
    "layer.hip": ["-ffp-contract=off"],
    "gemv.hip": ["-ffp-contract=off"],
}


# Kernel (mangled-name substring) -> allowed scratch bytes per lane.  The
# dK/dV kernel keeps a few loop-invariant mask values in scratch, reloaded only
# on tiles that need the mask.
SCRATCH_LIMITS = {
    "fwd128_kernel": 0,
    "dq128_kernel": 0,
    "dkdv128_kernel": 64,
    "dqds128_kernel": 0,
    "decode128_kernel": 0,
    "rmsnorm_kernel": 0,
}

# "Function Name: <kernel>" starts a kernel's block; then "<field> [unit]: value".
_REMARK = re.compile(r"remark:\s+(?:Function Name: (\S+)|(\w[\w ]*?)(?: \[[^\]]*\])?: (\S+)) \[-Rpass")


def _resource_usage(stderr: str) -> dict[str, dict[str, str]]:
    """Parses -Rpass-analysis=kernel-resource-usage remarks: kernel -> {field: value}."""
    out: dict[str, dict[str, str]] = {}
    cur = None
    for line in stderr.splitlines():
        m = _REMARK.search(line)
        if not m:
            continue
        if m.group(1):
            cur = m.group(1)
            out[cur] = {}
        elif cur is not None:
            out[cur][m.group(2).strip()] = m.group(3)
    return out


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found; the HIP toolchain is required to build")
    return exe


def _compile(src: Path) -> tuple[Path, dict[str, dict[str, str]]]:
    obj = BUILD / (src.name + ".o")
    remarks = ["-Rpass-analysis=kernel-resource-usage"] if src.suffix == ".hip" else []
    cmd = [hipcc(), *COMMON_FLAGS, *EXTRA_FLAGS.get(src.name, []), *remarks, "-c", str(src),
           "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return obj, _resource_usage(res.stderr)


def _check_resources(usage: dict[str, dict[str, str]]) -> None:
    lines = []
    for name in sorted(usage):
        f = usage[name]
        lines.append(f"{name}: VGPRs {f.get('VGPRs')} AGPRs {f.get('AGPRs')} "
                     f"scratch {f.get('ScratchSize')} B/lane occupancy {f.get('Occupancy')} "
                     f"waves/SIMD LDS {f.get('LDS Size')} B")
    (BUILD / "resource_usage.txt").write_text("\n".join(lines) + "\n")
    for key, limit in SCRATCH_LIMITS.items():
        hits = [n for n in usage if key in n]
        if not hits:
            raise RuntimeError(f"resource report has no kernel matching {key!r}")
        for n in hits:
            scratch = int(usage[n].get("ScratchSize", "0"))
            if scratch > limit:
                raise RuntimeError(f"{n} uses {scratch} bytes/lane of scratch (limit {limit}); "
                                   "see _build/resource_usage.txt")


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile every source in csrc/ and link the shared library; returns its path."""
    BUILD.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    sources = sorted([*CSRC.glob("*.hip"), *CSRC.glob("*.cpp")])
    jobs = jobs or min(len(sources), os.cpu_count() or 1, 16)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        results = list(ex.map(_compile, sources))
    objs = [obj for obj, _ in results]
    usage: dict[str, dict[str, str]] = {}
    for _, u in results:
        usage.update(u)
    _check_resources(usage)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}", file=sys.stderr)
    return LIB


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=None)
    args = ap.parse_args()
    build(args.jobs, verbose=True)


if __name__ == "__main__":
    main()
