"""Build ``libmk_mixtral.so`` for gfx950 with hipcc (in-tree, no JIT cache).

``python epic-kernel_amd/build.py`` or ``__graft_entry__.build()``.

Flags: ``-Xclang -target-feature -Xclang -packed-fp32-ops`` keeps the
compiler from emitting packed-fp32 VALU instructions; the host pass warns that
it does not know the feature, which is harmless.  The AMDGPU atomic optimizer
is off: all atomics are single-lane, and its wave-aggregated rewrite would
force a wait for each work-claim atomic right where it is issued.  ``MK_THREADS`` (workgroup
size) and ``MK_NT_LOADS`` (non-temporal weight loads) are tuning knobs.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parent
SRC = HERE / "csrc" / "mk_mixtral.hip"
OUT = HERE / "libmk_mixtral.so"
ARCH = os.environ.get("MK_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found")


def build(out: Path = OUT, defines: dict | None = None, verbose: bool = False) -> Path:
    cmd = [
        hipcc(),
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        # every atomic in the kernel is issued by one lane; the wave-aggregating
        # rewrite would broadcast each result right after the atomic and so
        # stall the work-claiming look-ahead on the atomic's round trip
        "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
        f"-I{REPO / 'include'}",
    ]
    for k, v in (defines or {}).items():
        cmd.append(f"-D{k}={v}")
    tmp = out.with_name(out.name + ".tmp")
    cmd += ["-o", str(tmp), str(SRC)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed ({res.returncode}) building {out.name}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
