"""Build ``liblogitfill_amd.so`` in-tree with hipcc for gfx950.

Every ``csrc/*.hip`` file is compiled to an object under ``logitfill_amd/_build``
and linked into ``logitfill_amd/liblogitfill_amd.so``; the C ABI is declared in
``include/logitfill_amd.h``.  Run ``python -m logitfill_amd.build``.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "liblogitfill_amd.so"
ARCH = os.environ.get("LOGITFILL_AMD_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 (hipcc's host pass warns that it
# does not know the feature; the device pass applies it).
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-result",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-gpu-flush-denormals-to-zero",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-mcode-object-version=5",
    f"-I{PKG.parent / 'include'}",
]


# Per-file additions.  decode_mfma.hip: the machine scheduler's max-ILP strategy, measured
# 82.9-83.0 -> 80.7-81.2 us per c2 layer-step (same box; the page compress, built with it,
# got slower, 121 -> 136 us, so it stays with the default), and the scheduler's own register
# pressure trackers (81.6-81.8 -> 80.6-80.8 us in a second same-box A/B).
_ILP = ["-mllvm", "-amdgpu-sched-strategy=max-ilp", "-mllvm", "-amdgpu-use-amdgpu-trackers=1"]
# decode_reduce.hip takes the same (c1 22.40-22.41 -> 22.31-22.33, c2 within 0.1-0.6 us lower).
# pack.hip: the trackers alone (c3 at targets 3.0 / 4.0 127.3-128.1 -> 126.4-126.9 and
# 129.0-129.6 -> 128.1-128.4 us, 2.5 unchanged; with max-ILP it was slower, see above).
FILE_FLAGS = {
    "decode_mfma.hip": _ILP,
    "decode_reduce.hip": _ILP,
    "pack.hip": ["-mllvm", "-amdgpu-use-amdgpu-trackers=1"],
}


def _compile(src: Path) -> tuple[Path, str]:
    obj = BUILD / (src.stem + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    log = "\n".join(
        line for line in (proc.stdout + proc.stderr).splitlines()
        if "packed-fp32-ops" not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{log}")
    return obj, log


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile all sources and link the shared library; returns its path."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    jobs = jobs or min(len(sources), max(1, (os.cpu_count() or 2) // 2), 8)
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        results = list(pool.map(_compile, sources))
    for obj, log in results:
        if verbose and log.strip():
            print(f"[{obj.name}]\n{log}", file=sys.stderr)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-mcode-object-version=5", "-shared", "-fPIC", "-o", str(tmp),
           *[str(o) for o, _ in results]]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}{proc.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    path = build(verbose=True)
    print(path)
