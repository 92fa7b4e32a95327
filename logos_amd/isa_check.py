"""Build-time check of the generated gfx950 code: wide vector-memory stores.

A store of more than 8 bytes (``*_store_dwordx3`` / ``*_store_dwordx4``)
reads its data registers after it issues.  The gfx940-family rule, which
LLVM's hazard recognizer applies to gfx950, is two wait states between such
a store and a VALU instruction that writes one of its data registers; a
rewrite inside that window can store the new value instead of the old.
This build keeps twice that (WINDOW = 4): the compiler's own spacing is
exactly two wait states at some stores, and those stores go through
store16_hold (logos_amd/csrc/vedic_common.hpp), which holds the registers
for four.
``scan()`` disassembles every code object in the library and reports each
wide store whose data registers a VALU (or MFMA) instruction writes within
``window`` wait states on any path from the store (each instruction counts
one wait state, ``s_nop N`` counts N + 1; branches are followed to their
targets, conditional ones both ways).

Used by ``build.build_library`` (the build fails on any finding) and by
tests/test_isa_check.py.
"""
from __future__ import annotations

import os
import re
import shutil
import subprocess
import tempfile

LLVM_BIN = "/opt/rocm/llvm/bin"
BUNDLE_MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"
RULE = 2    # wait states the gfx940 family needs
WINDOW = 4  # wait states this build keeps: twice the rule (store16_hold in vedic_common.hpp)

_STORE = re.compile(r"^(buffer|global|flat|scratch)_store_dwordx([34])\b\s+(.*)$")
_FUNC = re.compile(r"^[0-9a-f]+ <(.+)>:$")
_REG = re.compile(r"^([va])(\d+)$")
_RANGE = re.compile(r"^([va])\[(\d+):(\d+)\]$")


def _regs(tok: str) -> set:
    tok = tok.strip()
    m = _RANGE.match(tok)
    if m:
        return {(m.group(1), r) for r in range(int(m.group(2)), int(m.group(3)) + 1)}
    m = _REG.match(tok)
    return {(m.group(1), int(m.group(2)))} if m else set()


def _store_data(kind: str, ops: str) -> set:
    parts = [p.strip() for p in ops.split(",")]
    # buffer_store vdata, vaddr, srsrc, soffset; global/flat/scratch_store vaddr, vdata, ...
    tok = parts[0] if kind == "buffer" else (parts[1] if len(parts) > 1 else "")
    return _regs(tok.split()[0] if tok else "")


def _tool(name: str) -> str:
    p = os.path.join(LLVM_BIN, name)
    if os.path.exists(p):
        return p
    q = shutil.which(name)
    if q:
        return q
    raise RuntimeError(f"{name} not found: the code check needs the ROCm LLVM tools")


def disassemble(lib: str) -> list[str]:
    """Disassembly text of every gfx950 code object bundled in `lib` (a
    shared library or object file built by hipcc)."""
    texts = []
    with tempfile.TemporaryDirectory() as tmp:
        fat = os.path.join(tmp, "fatbin")
        subprocess.run(["objcopy", "--dump-section", f".hip_fatbin={fat}", lib, os.path.join(tmp, "copy")],
                       check=True, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)
        data = open(fat, "rb").read()
        starts = [m.start() for m in re.finditer(re.escape(BUNDLE_MAGIC), data)]
        for n, s in enumerate(starts):
            e = starts[n + 1] if n + 1 < len(starts) else len(data)
            piece = os.path.join(tmp, f"b{n}.bin")
            with open(piece, "wb") as f:
                f.write(data[s:e])
            co = os.path.join(tmp, f"b{n}.co")
            r = subprocess.run([_tool("clang-offload-bundler"), "--unbundle", "--type=o", f"--input={piece}",
                                f"--targets={TARGET}", f"--output={co}"], stdout=subprocess.PIPE,
                               stderr=subprocess.STDOUT, text=True)
            if r.returncode != 0 or not os.path.exists(co) or os.path.getsize(co) == 0:
                continue
            r = subprocess.run([_tool("llvm-objdump"), "-d", "--mcpu=gfx950", "--no-show-raw-insn", co],
                               stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, check=True)
            texts.append(r.stdout)
    return texts


_ADDR = re.compile(r"//\s*([0-9A-Fa-f]+):")


def _instructions(text: str):
    """(function, address, instruction text) in order."""
    func = "?"
    for line in text.splitlines():
        t = line.strip()
        m = _FUNC.match(t)
        if m:
            func = m.group(1)
            continue
        a = _ADDR.search(t)
        if not a or t.startswith(";"):
            continue
        ins = t.split("//")[0].strip()
        if ins:
            yield func, int(a.group(1), 16), ins


def _successors(ins, i, at):
    """Indices of the instructions that can follow instruction i."""
    t = ins[i][2]
    op = t.split()[0]
    if op in ("s_endpgm", "s_setpc_b64", "s_trap"):
        return []
    if op.startswith("s_branch") or op.startswith("s_cbranch"):
        imm = int(t.split()[1], 0)
        imm = imm - 0x10000 if imm >= 0x8000 else imm
        tgt = at.get(ins[i][1] + 4 + 4 * imm)
        out = [] if tgt is None else [tgt]
        if op.startswith("s_cbranch") and i + 1 < len(ins):
            out.append(i + 1)
        return out if (tgt is not None or op.startswith("s_cbranch")) else [None]
    return [i + 1] if i + 1 < len(ins) else []


def scan_text(text: str, window: int = WINDOW):
    """(stores, findings) for one disassembly; a finding is
    (function, store, instruction, wait states before it), every path of
    straight-line code and branches followed for `window` wait states."""
    ins = list(_instructions(text))
    at = {a: k for k, (_, a, _) in enumerate(ins)}
    stores, findings = 0, []
    for i, (func, _, t) in enumerate(ins):
        m = _STORE.match(t)
        if not m:
            continue
        stores += 1
        data = _store_data(m.group(1), m.group(3))
        todo = [(j, 0) for j in _successors(ins, i, at)]  # (instruction, wait states since the store)
        seen = set()
        while todo:
            j, ws = todo.pop()
            if ws >= window or (j, ws) in seen:
                continue
            seen.add((j, ws))
            if j is None:  # a branch whose target is not in this code object
                findings.append((func, t, "<unresolved branch>", ws))
                continue
            u = ins[j][2]
            if u.startswith("v_"):
                parts = u.split(None, 1)
                dst = parts[1].split(",")[0] if len(parts) > 1 else ""
                if _regs(dst) & data:
                    findings.append((func, t, u, ws))
                    continue
            n = re.match(r"s_nop\s+(0x[0-9a-fA-F]+|\d+)", u)
            cost = int(n.group(1), 0) + 1 if n else 1
            todo += [(k, ws + cost) for k in _successors(ins, j, at)]
    return stores, findings


def scan(lib: str, window: int = WINDOW):
    """(wide stores, findings) over every code object of `lib`."""
    total, found = 0, []
    for text in disassemble(lib):
        s, f = scan_text(text, window)
        total += s
        found += f
    return total, found


def main() -> None:
    import sys

    lib = sys.argv[1] if len(sys.argv) > 1 else os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                                              "liblogos_vedic.so")
    total, found = scan(lib)
    for func, st, u, ws in found:
        print(f"{func}: {st} ; {u} after {ws} wait states")
    print(f"{total} wide stores, {len(found)} with a data register rewritten within {WINDOW} wait states")
    raise SystemExit(1 if found else 0)


if __name__ == "__main__":
    main()
