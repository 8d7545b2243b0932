"""Static checks on the gfx950 code object this package builds.

Some pipelines issue LDS DMA (``buffer_load_dword[x4] ... lds``) as inline
assembly that the compiler's wait-count pass does not track (``lds_dma<B,
true>`` and ``lds_store16`` in ``csrc/mfma_pipe.h``). They order every read of
DMA-written LDS with their own ``s_waitcnt`` and barriers, which holds only
while the compiler issues no vector memory operations of its own inside their
loops; a spill reload there would bring its own wait and break that ordering
without any error. Inline assembly also gets no hazard padding from the
compiler. ``check_code_object`` therefore rejects

* scratch use (a non-zero private segment, SGPR or VGPR spills, or any
  ``scratch_*`` instruction) in a kernel that issues untracked LDS DMA (names
  in ``UNTRACKED_DMA_KERNELS``: the packed-weight MoE projections, whose DMA
  comes from ``csrc/w4pk.h``);

and, in every kernel that contains an LDS DMA,

* an LDS DMA fewer than 1 wait state after the SALU write of M0 it uses;
* an LDS DMA fewer than 5 wait states after a VALU write of an SGPR it reads
  (buffer resource or offset).

The wait states are the gfx9 hazard table's (an instruction counts one,
``s_nop N`` counts N + 1). The input is a code object built here from this
repository's own sources.
"""
from __future__ import annotations

import re
import subprocess
from dataclasses import dataclass, field
from pathlib import Path

LLVM_BIN = Path("/opt/rocm/llvm/bin")
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"

# Kernels whose LDS DMA is the inline-assembly form (the compiler's wait pass
# does not see it). Substrings of the mangled names.
UNTRACKED_DMA_KERNELS = ("moe_gate_up_pk_kernel", "moe_down_pk_kernel")

M0_WAIT = 1
VALU_SGPR_WAIT = 5

_LABEL = re.compile(r"^[0-9a-f]+ <(?P<name>[^>]+)>:\s*$")
_DMA = re.compile(r"^buffer_load_(dword|dwordx4|ubyte|ushort|sbyte|sshort)\b.*\blds\b")
_SREG = re.compile(r"\bs\[(\d+):(\d+)\]|\bs(\d+)\b|\b(vcc)\b|\b(m0)\b")


class CodeObjectError(RuntimeError):
    """A kernel of the built library breaks a rule its inline assembly relies on."""


@dataclass
class KernelReport:
    name: str
    dma: int = 0
    scratch_ops: int = 0
    private_segment: int = 0
    spills: int = 0
    problems: list = field(default_factory=list)


def _tool(name: str) -> str:
    path = LLVM_BIN / name
    return str(path) if path.exists() else name


def _run(cmd) -> str:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise CodeObjectError(f"{cmd[0]} failed: {proc.stderr.strip()}")
    return proc.stdout


def extract_device_code(binary: Path, out: Path) -> Path:
    """The gfx950 code object bundled in a host object or shared library."""
    out = Path(out)
    fatbin = out.with_suffix(".fatbin")
    _run([_tool("llvm-objcopy"), f"--dump-section=.hip_fatbin={fatbin}", str(binary), str(out.with_suffix(".host"))])
    _run([_tool("clang-offload-bundler"), "--unbundle", "--type=o", f"--input={fatbin}", f"--targets={TARGET}",
          f"--output={out}"])
    fatbin.unlink(missing_ok=True)
    out.with_suffix(".host").unlink(missing_ok=True)
    return out


def _sregs(text: str) -> set:
    regs = set()
    for m in _SREG.finditer(text):
        if m.group(1) is not None:
            regs.update(f"s{i}" for i in range(int(m.group(1)), int(m.group(2)) + 1))
        elif m.group(3) is not None:
            regs.add(f"s{m.group(3)}")
        elif m.group(4):
            regs.update(("vcc",))
        else:
            regs.add("m0")
    return regs


def _operands(inst: str) -> list:
    parts = inst.split(None, 1)
    if len(parts) < 2:
        return []
    ops, depth, cur = [], 0, ""
    for ch in parts[1]:
        if ch == "[":
            depth += 1
        elif ch == "]":
            depth -= 1
        if ch == "," and depth == 0:
            ops.append(cur.strip())
            cur = ""
        else:
            cur += ch
    if cur.strip():
        ops.append(cur.strip())
    return ops


_CARRY_OUT = re.compile(r"^v_(add|sub|subrev|addc|subb|subbrev)_co_u32|^v_mad_(u64_u32|i64_i32)|^v_div_scale")


def _valu_sgpr_writes(inst: str) -> set:
    """SGPRs (and vcc) a VALU instruction writes."""
    op = inst.split(None, 1)[0]
    ops = _operands(inst)
    if not op.startswith("v_") or not ops:
        return set()
    if op.startswith(("v_readfirstlane", "v_readlane")):
        return _sregs(ops[0])
    if op.startswith(("v_cmp", "v_cmpx")):
        return {"vcc"} if op.endswith("_e32") else _sregs(ops[0])
    if _CARRY_OUT.match(op):
        if op.endswith("_e32"):
            return {"vcc"}
        return _sregs(ops[1]) if len(ops) > 1 else set()
    return set()


def _wait_states(inst: str) -> int:
    if inst.startswith("s_nop"):
        ops = _operands(inst)
        return int(ops[0], 0) + 1 if ops else 1
    return 1


def _dma_sgpr_reads(inst: str) -> set:
    ops = _operands(inst)
    regs = set()
    for o in ops[1:]:
        regs |= _sregs(o)
    return regs


def _check_kernel(name: str, insts: list, meta: dict) -> KernelReport:
    rep = KernelReport(name)
    rep.private_segment = meta.get("private_segment_fixed_size", 0)
    rep.spills = meta.get("sgpr_spill_count", 0) + meta.get("vgpr_spill_count", 0)
    for i, inst in enumerate(insts):
        if inst.startswith("scratch_"):
            rep.scratch_ops += 1
        if not _DMA.match(inst):
            continue
        rep.dma += 1
        reads = _dma_sgpr_reads(inst)
        waits = 0
        m0_seen = False
        for j in range(i - 1, -1, -1):
            prev = insts[j]
            if not m0_seen and re.match(r"^s_\w+\s+m0\b", prev):
                m0_seen = True
                if waits < M0_WAIT:
                    rep.problems.append(f"LDS DMA {waits} wait states after the M0 write: {prev!r} -> {inst!r}")
            hit = _valu_sgpr_writes(prev) & reads
            if hit and waits < VALU_SGPR_WAIT:
                rep.problems.append(
                    f"LDS DMA reads {sorted(hit)} {waits} wait states after a VALU write: {prev!r} -> {inst!r}")
            waits += _wait_states(prev)
            if waits >= VALU_SGPR_WAIT and m0_seen:
                break
            if prev.startswith(("s_endpgm", "s_branch", "s_cbranch", "s_setpc")):
                break
    if rep.dma and any(k in name for k in UNTRACKED_DMA_KERNELS):
        if rep.private_segment:
            rep.problems.append(f"private segment of {rep.private_segment} bytes")
        if rep.spills:
            rep.problems.append(f"{rep.spills} register spills")
        if rep.scratch_ops:
            rep.problems.append(f"{rep.scratch_ops} scratch instructions")
    return rep


def _metadata(code_object: Path) -> dict:
    notes = _run([_tool("llvm-readelf"), "--notes", str(code_object)])
    meta, cur = {}, None
    for line in notes.splitlines():
        s = line.strip()
        m = re.match(r"^-?\s*\.name:\s+(\S+)", s)
        if m:
            cur = meta.setdefault(m.group(1), {})
            continue
        m = re.match(r"^-?\s*\.(private_segment_fixed_size|sgpr_spill_count|vgpr_spill_count):\s+(\d+)", s)
        if m and cur is not None:
            cur[m.group(1)] = int(m.group(2))
    return meta


def check_code_object(code_object: Path) -> list:
    """Reports for every kernel of a gfx950 code object; raises CodeObjectError
    listing every kernel with an LDS DMA that breaks a rule above."""
    meta = _metadata(code_object)
    dis = _run([_tool("llvm-objdump"), "-d", "--no-show-raw-insn", str(code_object)])
    kernels, name, insts = [], None, []
    for line in dis.splitlines():
        m = _LABEL.match(line)
        if m:
            if name is not None:
                kernels.append((name, insts))
            name, insts = m.group("name"), []
            continue
        s = line.split("//")[0].strip()
        if name is not None and s:
            insts.append(s)
    if name is not None:
        kernels.append((name, insts))
    reports = [_check_kernel(n, ins, meta.get(n, {})) for n, ins in kernels]
    bad = [r for r in reports if r.problems]
    if bad:
        lines = []
        for r in bad:
            lines.append(f"{r.name}:")
            lines.extend(f"  {p}" for p in r.problems[:8])
        raise CodeObjectError("kernels with LDS DMA break their scratch/hazard rules:\n" + "\n".join(lines))
    return reports


def check_binary(binary: Path, workdir: Path) -> list:
    """check_code_object on the device code of a host object or shared library."""
    workdir = Path(workdir)
    workdir.mkdir(parents=True, exist_ok=True)
    co = extract_device_code(binary, workdir / (Path(binary).stem + ".gfx950.co"))
    return check_code_object(co)
