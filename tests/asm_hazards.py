"""Wait-state check for inline-asm MFMAs in gfx950 assembly built from this repository's kernels.

The pipelined prefill kernel issues some MFMAs as inline asm (to pin O and Q^T in AGPRs).  The
compiler's hazard recognizer does not look inside inline asm, so it inserts no wait states for
those MFMAs: an instruction the compiler adds by itself -- above all a register copy
(v_accvgpr_mov / v_accvgpr_read) that joins two control-flow paths -- may read an MFMA result
while the MFMA is still writing it, or overwrite a register an in-flight MFMA still reads as
its accumulator input.  This module finds such accesses by data flow over the basic blocks of
each kernel: for every register written (or read as SrcC) by an inline-asm MFMA it tracks the
minimum number of wait states that have passed on any path, and reports a non-MFMA instruction
that touches the register before `need` wait states have passed.

Counting is conservative: every instruction is one wait state, `s_nop N` is N + 1; stalls the
hardware adds are not counted.  `need` defaults to 18 (the largest requirement the CDNA3/CDNA4
ISA lists for a VALU access after a 16-pass XDL op; a 32x32x16 f16 MFMA on gfx950 needs fewer).
"""
from __future__ import annotations

import re
from dataclasses import dataclass, field

_REG = re.compile(r"\b([av])\[(\d+):(\d+)\]|\b([av])(\d+)\b")
_WRITES_FIRST = re.compile(r"^(v_|ds_read|ds_load|global_load|buffer_load|flat_load|scratch_load)")


def _regs(text: str) -> set[str]:
    out: set[str] = set()
    for m in _REG.finditer(text):
        if m.group(1):
            out.update(f"{m.group(1)}{r}" for r in range(int(m.group(2)), int(m.group(3)) + 1))
        else:
            out.add(m.group(4) + m.group(5))
    return out


@dataclass
class Instr:
    line: int
    text: str
    op: str
    operands: list[str]
    in_asm: bool


@dataclass
class Block:
    label: str | None
    instrs: list[Instr] = field(default_factory=list)
    succ: list[str] = field(default_factory=list)
    falls_through: bool = True


def split_kernels(asm: str) -> dict[str, list[tuple[int, str]]]:
    """Kernel symbol -> its body lines (line number, text), from a `hipcc -S` listing."""
    kernels: dict[str, list[tuple[int, str]]] = {}
    cur = None
    for i, line in enumerate(asm.split("\n"), 1):
        m = re.match(r"^(_Z\w+):", line)
        if m:
            cur = m.group(1)
            kernels[cur] = []
            continue
        if cur is not None:
            if line.startswith("\t.size") or line.startswith(".Lfunc_end"):
                cur = None
                continue
            kernels[cur].append((i, line))
    return kernels


def _blocks(lines: list[tuple[int, str]]) -> list[Block]:
    blocks = [Block(None)]
    in_asm = False
    for no, line in lines:
        s = line.strip()
        if s.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if s.startswith(";;#ASMEND"):
            in_asm = False
            continue
        if not s or s.startswith(";") or (s.startswith(".") and not s.endswith(":")):
            continue
        if s.endswith(":"):
            blocks.append(Block(s[:-1]))
            continue
        s = s.split(";")[0].strip()
        op, _, rest = s.partition(" ")
        operands = [p.strip() for p in rest.split(",")] if rest else []
        cur = blocks[-1]
        cur.instrs.append(Instr(no, s, op, operands, in_asm))
        if op == "s_branch":
            cur.succ.append(operands[0])
            cur.falls_through = False
            blocks.append(Block(None))
        elif op.startswith("s_cbranch"):
            cur.succ.append(operands[0])
            blocks.append(Block(None))
        elif op in ("s_endpgm", "s_setpc_b64"):
            cur.falls_through = False
            blocks.append(Block(None))
    return [b for b in blocks if b.instrs or b.label]


def check_kernel(lines: list[tuple[int, str]], need: int = 18) -> list[str]:
    """Hazards (text lines) of one kernel; empty when every access waits long enough."""
    blocks = _blocks(lines)
    index = {b.label: i for i, b in enumerate(blocks) if b.label}
    preds: list[list[int]] = [[] for _ in blocks]
    for i, b in enumerate(blocks):
        for t in b.succ:
            if t in index:
                preds[index[t]].append(i)
        if b.falls_through and i + 1 < len(blocks):
            preds[i + 1].append(i)
    # state: (pending results, pending SrcC reads) as reg -> wait states elapsed
    State = tuple[dict[str, int], dict[str, int]]
    out_state: list[State | None] = [None] * len(blocks)
    hazards: dict[int, str] = {}

    def merge(states: list[State]) -> State:
        w: dict[str, int] = {}
        r: dict[str, int] = {}
        for sw, sr in states:
            for k, v in sw.items():
                w[k] = min(v, w.get(k, v))
            for k, v in sr.items():
                r[k] = min(v, r.get(k, v))
        return w, r

    def advance(st: State, n: int) -> State:
        sw, sr = st
        return ({k: v + n for k, v in sw.items() if v + n < need},
                {k: v + n for k, v in sr.items() if v + n < need})

    changed = True
    while changed:
        changed = False
        for i, b in enumerate(blocks):
            ins = [out_state[p] for p in preds[i] if out_state[p] is not None]
            st = merge(ins) if ins else ({}, {})
            for ins_ in b.instrs:
                if ins_.op == "s_nop":
                    st = advance(st, int(ins_.operands[0], 0) + 1)
                    continue
                if ins_.op.startswith("v_mfma"):
                    dst = _regs(ins_.operands[0])
                    srcab = _regs(",".join(ins_.operands[1:3]))
                    srcc = _regs(ins_.operands[3]) if len(ins_.operands) > 3 else set()
                    sw, sr = st
                    bad = srcab & set(sw)
                    if srcc & set(sw) and srcc != dst:
                        bad |= srcc & set(sw)
                    if bad:
                        hazards[ins_.line] = f"{ins_.line}: {ins_.text}  (reads {sorted(bad)[0]} too soon)"
                    st = advance(st, 1)
                    if ins_.in_asm:
                        sw, sr = st
                        sw = dict(sw)
                        sr = dict(sr)
                        for r in dst:
                            sw[r] = 0
                        for r in srcc:
                            sr[r] = 0
                        st = (sw, sr)
                    continue
                sw, sr = st
                touched = _regs(",".join(ins_.operands))
                hit = touched & set(sw)
                if _WRITES_FIRST.match(ins_.op) and ins_.operands:
                    hit |= _regs(ins_.operands[0]) & set(sr)
                if hit:
                    r = sorted(hit)[0]
                    waited = sw.get(r, sr.get(r))
                    hazards[ins_.line] = f"{ins_.line}: {ins_.text}  ({r} after {waited} wait states)"
                st = advance(st, 1)
            if out_state[i] != st:
                out_state[i] = st
                changed = True
    return [hazards[k] for k in sorted(hazards)]


def check_listing(asm: str, need: int = 18) -> dict[str, list[str]]:
    """Kernel symbol -> hazards, for every kernel of the listing that has inline-asm MFMAs."""
    out = {}
    for name, lines in split_kernels(asm).items():
        text = "\n".join(l for _, l in lines)
        if "ASMSTART" not in text or "v_mfma" not in text:
            continue
        out[name] = check_kernel(lines, need)
    return out
