"""The C ABI boundary without a GPU: the library loads, exports every entry
point include/*.h declares, the ctypes struct has the header's layout, and
host-side validation rejects bad calls before any HIP call is made."""

import ctypes
import re
import subprocess
from pathlib import Path

import pytest
import torch

import mk_mixtral
from megakernels_amd.mixtral.mk import interpret_with_mk
from megakernels_amd.mixtral.scheduler import make_globals
from megakernels_amd.mixtral.synthetic import SMALL, make_synthetic_mixtral
from megakernels_amd.scheduler import tensorize_instructions

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "mk_mixtral.h"
HEADERS = sorted((ROOT / "include").glob("*.h"))


@pytest.fixture(scope="module")
def lib():
    if not mk_mixtral.library_path().exists():
        import __graft_entry__

        __graft_entry__.build()
    return mk_mixtral.load_library()


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(mk_mixtral_\w+)\s*\(", text, re.M)))


def test_header_declares_entry_points():
    names = declared_functions()
    assert "mk_mixtral_launch" in names
    assert sorted(mk_mixtral.EXPORTED_SYMBOLS) == names


def all_declared_functions():
    names = set()
    for h in HEADERS:
        names |= set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(mk_\w+)\s*\(", h.read_text(), re.M))
    return sorted(names)


def test_library_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(mk_mixtral.library_path())],
                         capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    names = all_declared_functions()
    assert "mk_llama_launch" in names and "mk_mixtral_launch" in names
    for name in names:
        assert name in exported, name
        assert hasattr(lib, name)


def test_llama_header_entry_points_and_layout(tmp_path):
    import mk_llama

    text = (ROOT / "include" / "mk_llama.h").read_text()
    declared = sorted(set(re.findall(r"^\s*\w+\s*(mk_llama_\w+)\s*\(", text, re.M)))
    assert declared == sorted(mk_llama.EXPORTED_SYMBOLS)
    fields = [f for f, _ in mk_llama.MkLlamaGlobals._fields_]
    src = tmp_path / "layout.c"
    src.write_text(
        '#include <stddef.h>\n#include <stdio.h>\n#include "mk_llama.h"\nint main(void) {\n'
        '  printf("sizeof %zu\\n", sizeof(mk_llama_globals));\n'
        + "".join(f'  printf("{f} %zu\\n", offsetof(mk_llama_globals, {f}));\n' for f in fields)
        + "  return 0;\n}\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", f"-I{ROOT / 'include'}", str(src), "-o", str(exe)], check=True)
    lines = dict(l.split() for l in subprocess.run([str(exe)], capture_output=True, text=True, check=True)
                 .stdout.splitlines())
    assert int(lines.pop("sizeof")) == ctypes.sizeof(mk_llama.MkLlamaGlobals)
    for f in fields:
        assert int(lines[f]) == getattr(mk_llama.MkLlamaGlobals, f).offset, f


def test_llama_launch_validation_needs_no_gpu(lib):
    import mk_llama

    mk_llama.load_library()
    assert lib.mk_llama_abi_version() == mk_llama.ABI_VERSION
    assert lib.mk_llama_launch(None, None) == 1
    g = mk_llama.MkLlamaGlobals()
    g.struct_size = ctypes.sizeof(g)
    g.abi_version = 99
    assert lib.mk_llama_launch(ctypes.byref(g), None) == 1
    g.abi_version = mk_llama.ABI_VERSION
    assert lib.mk_llama_launch(ctypes.byref(g), None) == 1  # null tensors
    with pytest.raises(TypeError):
        mk_llama.mk_llama(1, 2, 3)
    args = [torch.empty(0)] * 16 + [torch.empty(4, dtype=torch.bfloat16)] + [torch.empty(0)] * 6
    with pytest.raises(ValueError, match="GPU"):
        mk_llama.build_llama_struct(*args, 0, 1.0, 1e-5, False)


def test_decode_tail_arguments_are_checked():
    """argmax_out / next_embed_weights: int64 output, an LM head to take the
    argmax of, and the embedding table only together with argmax_out."""
    out = torch.zeros((), dtype=torch.int64)
    emb = torch.zeros(8, 512, dtype=torch.bfloat16)
    dev = torch.device("cpu")
    assert mk_mixtral._decode_tail(None, None, False, dev, 512) == (None, None)
    assert mk_mixtral._decode_tail(out, emb, True, dev, 512) == (out.data_ptr(), emb.data_ptr())
    with pytest.raises(ValueError, match="needs argmax_out"):
        mk_mixtral._decode_tail(None, emb, True, dev, 512)
    with pytest.raises(ValueError, match="LM head"):
        mk_mixtral._decode_tail(out, None, False, dev, 512)
    with pytest.raises(TypeError):
        mk_mixtral._decode_tail(out.int(), None, True, dev, 512)
    with pytest.raises(ValueError, match=r"\[V, 1024\]"):
        mk_mixtral._decode_tail(out, emb, True, dev, 1024)


def test_struct_layout_matches_header(tmp_path):
    fields = [f for f, _ in mk_mixtral.MkMixtralGlobals._fields_]
    src = tmp_path / "layout.c"
    src.write_text(
        '#include <stddef.h>\n#include <stdio.h>\n#include "mk_mixtral.h"\nint main(void) {\n'
        '  printf("sizeof %zu\\n", sizeof(mk_mixtral_globals));\n'
        + "".join(f'  printf("{f} %zu\\n", offsetof(mk_mixtral_globals, {f}));\n' for f in fields)
        + "  return 0;\n}\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", f"-I{ROOT / 'include'}", str(src), "-o", str(exe)], check=True)
    lines = dict(l.split() for l in subprocess.run([str(exe)], capture_output=True, text=True, check=True)
                 .stdout.splitlines())
    assert int(lines.pop("sizeof")) == ctypes.sizeof(mk_mixtral.MkMixtralGlobals)
    for f in fields:
        assert int(lines[f]) == getattr(mk_mixtral.MkMixtralGlobals, f).offset, f


def test_version_and_error_strings(lib):
    assert lib.mk_mixtral_abi_version() == mk_mixtral.ABI_VERSION
    for code in (0, 1, 2, 3, 4, 16, 17, 18, 19):
        assert lib.mk_mixtral_error_string(code)
    assert b"unknown" in lib.mk_mixtral_error_string(12345)


def test_tuning_overrides_are_reported_and_malformed_ones_ignored(lib, capfd, monkeypatch):
    """The measurement overrides are read from the environment once per
    process (mk_mixtral_reload_overrides reads them again): each one in
    effect is reported on stderr, a value that is not a whole number is
    ignored with a warning, and nothing is reported without them."""
    for name in ("MK_SPREAD", "MK_SPIN_SLEEP", "MK_TAIL", "MK_EARLY", "MK_PF", "MK_STAGE_ITEMS"):
        monkeypatch.delenv(name, raising=False)
    monkeypatch.setenv("MK_TAIL", "8")
    monkeypatch.setenv("MK_PF", " 0x2 ")
    monkeypatch.setenv("MK_EARLY", "4x")
    lib.mk_mixtral_reload_overrides()
    err = capfd.readouterr().err
    assert "measurement override MK_TAIL=8 in effect" in err
    assert "measurement override MK_PF=2 in effect" in err
    assert 'ignoring MK_EARLY="4x"' in err and "MK_EARLY=4" not in err
    for name in ("MK_TAIL", "MK_PF", "MK_EARLY"):
        monkeypatch.delenv(name)
    lib.mk_mixtral_reload_overrides()
    assert "mk_mixtral:" not in capfd.readouterr().err


def test_launch_validation_needs_no_gpu(lib):
    # a null struct and a struct of the wrong ABI are rejected before any HIP call
    assert lib.mk_mixtral_launch(None, None) == 1
    g = mk_mixtral.MkMixtralGlobals()
    g.struct_size = ctypes.sizeof(g)
    g.abi_version = 99
    assert lib.mk_mixtral_launch(ctypes.byref(g), None) == 1
    g.abi_version = mk_mixtral.ABI_VERSION
    assert lib.mk_mixtral_launch(ctypes.byref(g), None) == 1  # null tensors


def test_python_launcher_rejects_bad_arguments():
    model = make_synthetic_mixtral(SMALL, "cpu", 0)
    g = make_globals(model, sm_count=2)
    tensorize_instructions(g, [[], []])
    with pytest.raises(ValueError, match="GPU"):
        interpret_with_mk(g, mk_mixtral.mk_mixtral)
    with pytest.raises(TypeError):
        mk_mixtral.mk_mixtral(1, 2, 3)
    # hidden_states on the CPU: refused before the library is called
    args = [torch.empty(0)] * 17 + [torch.empty(4, dtype=torch.bfloat16)] + [torch.empty(0)] * 10
    with pytest.raises(ValueError, match="GPU"):
        mk_mixtral.build_globals_struct(*args, 0, 1.0, 1e-5, False)


def _asm(kernel, before_getpc, length, getpc=True):
    body = "\n".join(["\ts_mov_b32 s0, 0"] * before_getpc + (["\ts_getpc_b64 s[4:5]"] if getpc else []) +
                     ["\ts_endpgm"])
    return (f"\t.p2align\t8\n\t.type\t{kernel},@function\n{kernel}: ; @{kernel}\n; %bb.0:\n"
            f"\t; a comment\n{body}\n.Lfunc_end0:\n\t.size\t{kernel}, .Lfunc_end0-{kernel}\n"
            f"; codeLenInByte = {length}\n; NumVgprs: 10\n")


def test_build_reads_code_lengths_and_checks_the_entry_pc():
    """build.py's second compile hands each kernel's machine-code length to
    the host code, for the kernel's reads of its own code: the lengths come
    from the compiler's device assembly, and the build refuses a kernel that
    reads its program counter too far from its entry (the rounding down to
    the 256-byte-aligned entry would then be wrong) or not at all."""
    import build

    names = list(build.KERNELS)
    asm = "".join(_asm(k, 3, 1000 + i) for i, k in enumerate(names))
    assert build.code_lengths(asm) == {k: 1000 + i for i, k in enumerate(names)}
    far = "".join(_asm(k, build.MAX_INSNS_BEFORE_GETPC + 1 if i == 2 else 0, 64) for i, k in enumerate(names))
    with pytest.raises(RuntimeError, match="before s_getpc_b64"):
        build.code_lengths(far)
    missing = "".join(_asm(k, 0, 64, getpc=i != 1) for i, k in enumerate(names))
    with pytest.raises(RuntimeError, match="no s_getpc_b64"):
        build.code_lengths(missing)
    with pytest.raises(RuntimeError, match="no code length"):
        build.code_lengths("".join(_asm(k, 0, 64) for k in names[:-1]))


def test_build_reads_function_sizes_from_the_linked_object():
    """The prefetch bound is the kernel's symbol size in the linked device
    code object: a minimal ELF with a symbol table of two functions and one
    object reads back as the two functions' (address, size)."""
    import struct

    import build

    names = [b"", b"kern_a", b"kern_b", b"data_c"]
    strtab = b"\0".join(names) + b"\0"
    offs = [0]
    for n in names[1:]:
        offs.append(offs[-1] + len(names[len(offs) - 1]) + 1)
    syms = struct.pack("<IBBHQQ", 0, 0, 0, 0, 0, 0)
    syms += struct.pack("<IBBHQQ", offs[1], 0x12, 0, 1, 0x3100, 304572)   # FUNC
    syms += struct.pack("<IBBHQQ", offs[2], 0x12, 0, 1, 0x95900, 280704)  # FUNC
    syms += struct.pack("<IBBHQQ", offs[3], 0x11, 0, 1, 0x2000, 64)       # OBJECT
    head = bytearray(64)
    head[:6] = b"\x7fELF\x02\x01"
    str_off = 64
    sym_off = str_off + len(strtab)
    sh_off = sym_off + len(syms)
    struct.pack_into("<Q", head, 0x28, sh_off)
    struct.pack_into("<HHH", head, 0x3A, 64, 3, 0)
    sections = struct.pack("<IIQQQQIIQQ", 0, 0, 0, 0, 0, 0, 0, 0, 0, 0)
    sections += struct.pack("<IIQQQQIIQQ", 0, 3, 0, 0, str_off, len(strtab), 0, 0, 1, 0)   # SHT_STRTAB
    sections += struct.pack("<IIQQQQIIQQ", 0, 2, 0, 0, sym_off, len(syms), 1, 1, 8, 24)   # SHT_SYMTAB -> 1
    data = bytes(head) + strtab + syms + sections
    assert build.elf_functions(data) == {"kern_a": (0x3100, 304572), "kern_b": (0x95900, 280704)}
    with pytest.raises(RuntimeError):
        build.elf_functions(b"\x7fELF\x01\x01" + bytes(58))
