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
import struct
import subprocess
import sys
import tempfile
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


# Kernel symbol (as the compiler names it) -> the macro that carries its
# machine-code length into the host code (code_prefetch's bound).
KERNELS = {
    "_ZN12_GLOBAL__N_115mk_llama_kernelENS_7KParamsE": "MK_CODE_LEN_LLAMA",
    "_ZN12_GLOBAL__N_117mk_mixtral_kernelILi8ELb1EEEvNS_7KParamsE": "MK_CODE_LEN_E8_ATTN",
    "_ZN12_GLOBAL__N_117mk_mixtral_kernelILi0ELb1EEEvNS_7KParamsE": "MK_CODE_LEN_E0_ATTN",
    "_ZN12_GLOBAL__N_117mk_mixtral_kernelILi8ELb0EEEvNS_7KParamsE": "MK_CODE_LEN_E8",
    "_ZN12_GLOBAL__N_117mk_mixtral_kernelILi0ELb0EEEvNS_7KParamsE": "MK_CODE_LEN_E0",
}
# kernel_code_base() rounds the program counter down to the kernel's
# 256-byte-aligned entry, so its s_getpc_b64 must sit in the first 256 bytes:
# at most this many instructions (12 bytes at most each) before it.
MAX_INSNS_BEFORE_GETPC = 20


def code_lengths(asm: str) -> dict[str, int]:
    """Machine-code length of every kernel in the device assembly, and a
    check that each kernel reads its program counter within its first 256
    bytes."""
    lengths: dict[str, int] = {}
    current = None
    before = None  # instructions seen before s_getpc_b64 in the current kernel
    for line in asm.splitlines():
        if "codeLenInByte" in line:
            if current is not None:
                if before is not None:
                    raise RuntimeError(f"{current}: no s_getpc_b64 near the entry")
                lengths[current] = int(line.split("=")[1])
            current = None
            continue
        head = line.split(";", 1)[0].strip()
        if not head or head.startswith("."):
            continue
        if head.endswith(":"):
            if head[:-1] in KERNELS:
                current, before = head[:-1], 0
            continue
        if current is not None and before is not None:
            if head.startswith("s_getpc_b64"):
                if before > MAX_INSNS_BEFORE_GETPC:
                    raise RuntimeError(f"{current}: {before} instructions before s_getpc_b64")
                before = None
            else:
                before += 1
    missing = set(KERNELS) - set(lengths)
    if missing:
        raise RuntimeError(f"no code length for {sorted(missing)}")
    return lengths


def elf_functions(data: bytes) -> dict[str, tuple[int, int]]:
    """(address, size) of every function symbol of a 64-bit little-endian
    ELF file (the linked device code object)."""
    if data[:4] != b"\x7fELF" or data[4] != 2 or data[5] != 1:
        raise RuntimeError("not a 64-bit little-endian ELF file")
    shoff, = struct.unpack_from("<Q", data, 0x28)
    shentsize, shnum = struct.unpack_from("<HH", data, 0x3A)
    sections = [struct.unpack_from("<IIQQQQIIQQ", data, shoff + i * shentsize) for i in range(shnum)]
    out: dict[str, tuple[int, int]] = {}
    for sec in sections:
        if sec[1] != 2:  # SHT_SYMTAB
            continue
        strtab = sections[sec[6]]
        for off in range(sec[4], sec[4] + sec[5], 24):
            name_off, info, _other, _shndx, value, size = struct.unpack_from("<IBBHQQ", data, off)
            if info & 0xF != 2:  # STT_FUNC
                continue
            start = strtab[4] + name_off
            name = data[start:data.index(b"\0", start)].decode()
            out[name] = (value, size)
    return out


def compile_once(out: Path, defines: dict, verbose: bool) -> dict[str, int]:
    """One hipcc compile of the library into `out`; returns the kernels'
    machine-code lengths: the sizes of their symbols in the linked device
    code object of that same compile (the assembly's codeLenInByte is the
    compiler's estimate before branch relaxation and can exceed them by a
    few hundred bytes), after checking that each kernel starts on a 256-byte
    boundary and reads its program counter within its first 256 bytes."""
    cmd = [
        hipcc(),
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-save-temps",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        # every atomic in the kernel is issued by one lane; the wave-aggregating
        # rewrite would broadcast each result right after the atomic and so
        # stall the work-claiming look-ahead on the atomic's round trip
        "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
        f"-I{REPO / 'include'}",
    ]
    for k, v in defines.items():
        cmd.append(f"-D{k}={v}")
    cmd += ["-o", str(out), str(SRC)]
    if verbose:
        print(" ".join(cmd), flush=True)
    with tempfile.TemporaryDirectory(prefix="mk_build_") as tmp:
        res = subprocess.run(cmd, capture_output=True, text=True, cwd=tmp)
        if res.returncode != 0:
            sys.stderr.write(res.stdout + res.stderr)
            raise RuntimeError(f"hipcc failed ({res.returncode}) building {out.name}")
        # the device assembly hipcc keeps with -save-temps
        # (<stem>-hip-amdgcn-amd-amdhsa-<arch>.s with ROCm 7)
        asms = sorted(Path(tmp).glob(f"*amdgcn*{ARCH}*.s"))
        objs = sorted(Path(tmp).glob(f"*amdgcn*{ARCH}*.out"))
        if len(asms) != 1 or len(objs) != 1:
            raise RuntimeError(f"expected one device assembly and one linked device object from -save-temps, "
                               f"found {[a.name for a in asms + objs]}")
        estimates = code_lengths(asms[0].read_text())
        funcs = elf_functions(objs[0].read_bytes())
        lengths = {}
        for name, estimate in estimates.items():
            if name not in funcs:
                raise RuntimeError(f"{name} is not in the linked device code object")
            addr, size = funcs[name]
            if addr % 256 or not 0 < size <= estimate:
                raise RuntimeError(f"{name}: at {addr:#x}, {size} bytes (estimate {estimate})")
            lengths[name] = size
        return lengths


def build(out: Path = OUT, defines: dict | None = None, verbose: bool = False) -> Path:
    """Compile the library twice: the first compile measures each kernel's
    machine-code length, the second passes the lengths to the host code.
    The device code does not depend on them, so both compiles must give the
    same lengths (checked)."""
    defines = dict(defines or {})
    out = Path(out).resolve()  # the compiles run in a temporary directory
    tmp = out.with_name(out.name + ".tmp")
    first = compile_once(tmp, defines, verbose)
    lens = {KERNELS[k]: n for k, n in first.items()}
    if verbose:
        print("machine-code bytes:", lens, flush=True)
    second = compile_once(tmp, {**defines, **lens}, verbose)
    if second != first:
        raise RuntimeError(f"device code changed between the two compiles: {first} vs {second}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
