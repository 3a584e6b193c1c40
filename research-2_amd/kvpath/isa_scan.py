"""Scan gfx950 assembly for uses of an inline-asm load's destination before the wait covering it.

The attention kernels issue some loads as inline asm the compiler does not track (global loads
into registers, LDS reads), each followed by an explicit s_waitcnt and an empty asm tying the
register. That is only correct while the compiler leaves the destination alone until the wait:
no copy of it (it would read the register before the data lands) and no reuse (the late data
would overwrite the new value).

The scan splits each kernel into basic blocks (at labels, at the compiler's `; %bb.N:` block
comments, and after every branch) and walks the control-flow graph from the entry, carrying the
outstanding vector-memory and LDS operations in issue order (`s_waitcnt vmcnt(N)` / `lgkmcnt(N)`
retire all but the newest N). States are propagated along every edge -- fall-through, taken
branches and loop back-edges -- until no block sees a new state, so a load issued at the end of a
loop body is still outstanding at the loop header. Any instruction that reads or writes a
register an outstanding inline-asm load will still write is reported.

The kernels choose between two waits, `if (more) wait(N); else wait(0);`, where `more` says the
next block's N loads were issued: wait for everything but those. The compiler lowers the pair
with a boolean in an SGPR pair (a branch around `s_waitcnt vmcnt(0); s_mov_b64 s[x:y], 0`, then
`s_andn2_b64 vcc, exec, s[x:y]` and `s_cbranch_vccnz` around `s_waitcnt vmcnt(N)`). The scan
treats such a pair as the one wait it stands for -- vmcnt(N) when more than N operations are
outstanding, vmcnt(0) otherwise -- and continues at the join. The choice of branch depends on
data the scan does not follow (whether the next block exists), so exploring both arms would
pair a wait(N) with a step that issued no further loads, or skip both waits: paths no execution
takes. What is checked is the compiler's handling of the destination registers. That the kernel
waits for the right block is not: a counted wait that keeps more than the next block's loads
reads, to the scan, like the last block's wait(0) (the parity tests cover the waits' counts).
Each path also carries the
SGPR pairs it set to a constant and what they make of vcc, so a branch those constants decide
follows only the edge it takes.
"""

from __future__ import annotations

import re
from dataclasses import dataclass, field

_RANGE = re.compile(r"\b([va])\[(\d+):(\d+)\]")
_SINGLE = re.compile(r"\b([va])(\d+)\b")
_SRANGE = re.compile(r"\bs\[(\d+):(\d+)\]")
_SSINGLE = re.compile(r"\bs(\d+)\b")
_LABEL = re.compile(r"^(\.?L[\w$.]+|_Z\S+):")
_BB_COMMENT = re.compile(r"^;\s*%bb\.\d+:")
_VMEM_LOAD = ("global_load", "buffer_load", "scratch_load", "flat_load")
_VMEM_OTHER = ("global_store", "buffer_store", "scratch_store", "flat_store", "global_atomic",
               "buffer_atomic")
_LGKM = ("ds_", "s_load", "s_buffer_load")
_MAX_VISITS = 200_000  # the walk gives up (and reports so) past this many block visits


def _regs(text: str) -> frozenset:
    out = set()
    for kind, lo, hi in _RANGE.findall(text):
        out |= {(kind, i) for i in range(int(lo), int(hi) + 1)}
    stripped = _RANGE.sub(" ", text)
    out |= {(kind, int(n)) for kind, n in _SINGLE.findall(stripped)}
    return frozenset(out)


def _sregs(text: str) -> frozenset:
    out = set()
    for lo, hi in _SRANGE.findall(text):
        out |= set(range(int(lo), int(hi) + 1))
    out |= {int(n) for n in _SSINGLE.findall(_SRANGE.sub(" ", text))}
    return frozenset(out)


def _retire(pending: tuple, keep: int) -> tuple:
    return pending[len(pending) - keep:] if keep < len(pending) else pending


@dataclass
class _Instr:
    text: str
    op: str
    operands: str
    in_asm: bool


@dataclass
class _Block:
    name: str
    instrs: list = field(default_factory=list)
    fall: int | None = None    # fall-through successor
    taken: int | None = None   # branch target
    branch: str = ""           # the block's closing branch op, if any


def _blocks(lines: list[str]) -> list[_Block]:
    blocks = [_Block("entry")]
    index: dict[str, int] = {}
    targets: list[tuple[int, str]] = []
    ends: set[int] = set()  # blocks with no fall-through (s_branch, s_endpgm, s_setpc)
    in_asm = False

    def start(name: str) -> None:
        # A block with no instructions yet takes the new label as well (labels that follow one
        # another, or a label right after a branch, name one block).
        if blocks[-1].instrs:
            blocks.append(_Block(name))
        else:
            blocks[-1].name = name

    for line in lines:
        s = line.strip()
        if s.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if s.startswith(";;#ASMEND"):
            in_asm = False
            continue
        m = _LABEL.match(s)
        if m or _BB_COMMENT.match(s):
            start(m.group(1) if m else s.split()[1].rstrip(":"))
            index[blocks[-1].name] = len(blocks) - 1
            continue
        if not s or s.startswith((";", ".")):
            continue
        op = s.split()[0]
        blocks[-1].instrs.append(_Instr(s, op, s[len(op):].split(";")[0], in_asm))
        here = len(blocks) - 1
        if op == "s_branch" or op.startswith("s_cbranch"):
            blocks[here].branch = op
            targets.append((here, s.split()[1]))
            if op == "s_branch":
                ends.add(here)
            start(f"after{here}")
        elif op.startswith("s_endpgm") or op.startswith("s_setpc"):
            ends.add(here)
            start(f"after{here}")
    for i, b in enumerate(blocks):
        if i not in ends and i + 1 < len(blocks):
            b.fall = i + 1
    for i, target in targets:
        blocks[i].taken = index.get(target)
    return blocks


def _track_constants(ins: _Instr, consts: dict) -> None:
    """Update the path's known SGPR-pair constants and vcc after one instruction (in place).
    Keys are SGPR-pair bases (the pair s[b:b+1]) and "vcc"; vcc is "zero" or "nonzero"."""
    op, operands = ins.op, ins.operands
    args = [a.strip() for a in operands.split(",")]
    m = re.fullmatch(r"s\[(\d+):(\d+)\]", args[0]) if args and args[0] else None
    if op == "s_mov_b64" and m and len(args) == 2 and args[1] in ("-1", "0"):
        written = _sregs(args[0])
        for k in [k for k in consts if k != "vcc" and {k, k + 1} & written]:
            del consts[k]
        consts[int(m.group(1))] = int(args[1])
        return
    if op in ("s_andn2_b64", "s_and_b64") and len(args) == 3 and args[0] == "vcc" and \
            args[1] == "exec":
        m2 = re.fullmatch(r"s\[(\d+):(\d+)\]", args[2])
        value = consts.get(int(m2.group(1))) if m2 else None
        consts.pop("vcc", None)
        if value is not None:
            # exec is not zero on a path the wave executes scalar code on.
            flag_set = value == -1
            nonzero = (not flag_set) if op == "s_andn2_b64" else flag_set
            consts["vcc"] = "nonzero" if nonzero else "zero"
        return
    # Any other write: forget what it may overwrite (an SGPR named anywhere but as the source of
    # a store-like op may be written; vcc by any op naming it or by a VOPC compare).
    named = _sregs(operands)
    for k in [k for k in consts if k != "vcc" and {k, k + 1} & named]:
        del consts[k]
    if "vcc" in operands or op.startswith("v_cmp") or op.startswith("v_cmpx") or \
            op.endswith("_co_u32") or "vcc" in op:
        consts.pop("vcc", None)


def _only(block: _Block, *ops: str) -> bool:
    return [i.op for i in block.instrs] == list(ops)


def _wait_pair(blocks: list[_Block], bi: int) -> tuple[int, str, int] | None:
    """If block bi opens a compiled wait pair, (N, flag pair, join after the pair), else None."""
    b = blocks[bi]
    if not b.branch.startswith("s_cbranch") or b.fall is None or b.taken is None:
        return None
    for w0, j in ((b.fall, b.taken), (b.taken, b.fall)):
        wb, jb = blocks[w0], blocks[j]
        if not (_only(wb, "s_waitcnt", "s_mov_b64") and wb.fall == j and
                re.search(r"vmcnt\(0\)", wb.instrs[0].text) and
                re.fullmatch(r"\s*s\[\d+:\d+\],\s*0\s*", wb.instrs[1].operands)):
            continue
        flag = wb.instrs[1].operands.split(",")[0].strip()
        if not (_only(jb, "s_andn2_b64", "s_cbranch_vccnz") and
                [a.strip() for a in jb.instrs[0].operands.split(",")] == ["vcc", "exec", flag]):
            continue
        if jb.fall is None or not _only(blocks[jb.fall], "s_waitcnt") or \
                blocks[jb.fall].fall != jb.taken:
            continue
        m = re.search(r"vmcnt\((\d+)\)", blocks[jb.fall].instrs[0].text)
        if m and "lgkmcnt" not in blocks[jb.fall].instrs[0].text:
            return int(m.group(1)), flag, jb.taken
    return None


def scan(asm: str) -> dict[str, list[str]]:
    """-> {kernel symbol: [reports]} for every kernel in `asm`."""
    result = {}
    for chunk in re.split(r"\n(?=_Z\S*:)", asm):
        name = chunk.split(":", 1)[0].strip()
        if not name.startswith("_Z"):
            continue
        blocks = _blocks(chunk.split("\n")[1:])
        reports: dict[tuple[int, int], str] = {}
        if not any(i.in_asm and (i.op.startswith(_VMEM_LOAD) or i.op.startswith("ds_read"))
                   for b in blocks for i in b.instrs):
            result[name] = []  # no inline-asm load: nothing can be outstanding behind the compiler
            continue
        seen: list[set] = [set() for _ in blocks]
        work = [(0, (), (), ())]
        visits = 0
        while work:
            bi, vm, lgkm, const_items = work.pop()
            key = (vm, lgkm, const_items)
            if key in seen[bi]:
                continue
            seen[bi].add(key)
            visits += 1
            if visits > _MAX_VISITS:
                reports[(-1, -1)] = f"scan gave up after {_MAX_VISITS} block visits"
                break
            consts = dict(const_items)
            block = blocks[bi]
            for ii, ins in enumerate(block.instrs):
                s, op, operands = ins.text, ins.op, ins.operands
                if op == "s_waitcnt":
                    m = re.search(r"vmcnt\((\d+)\)", s)
                    if m:
                        vm = _retire(vm, int(m.group(1)))
                    m = re.search(r"lgkmcnt\((\d+)\)", s)
                    if m:
                        lgkm = _retire(lgkm, int(m.group(1)))
                    continue
                if op.startswith(("s_endpgm", "s_setpc", "s_branch", "s_cbranch")):
                    continue
                touched = _regs(operands)
                live = set()
                for from_asm, regs in vm + lgkm:
                    if from_asm:
                        live |= regs
                clash = touched & live
                if clash:
                    reports.setdefault(
                        (bi, ii), f"{s}  <- outstanding inline-asm load into {sorted(clash)[:4]}")
                dest = operands.split(",")[0]
                is_dma = "_lds" in op or " lds" in f" {operands}"  # to LDS: no register destination
                # Only inline-asm loads need their destinations; the compiler's own only count.
                if op.startswith(_VMEM_LOAD) and not is_dma:
                    vm = vm + ((ins.in_asm, _regs(dest) if ins.in_asm else frozenset()),)
                elif op.startswith(_VMEM_OTHER) or op.startswith(_VMEM_LOAD):
                    vm = vm + ((ins.in_asm, frozenset()),)
                elif op.startswith("ds_read") or op.startswith("ds_load"):
                    lgkm = lgkm + ((ins.in_asm, _regs(dest) if ins.in_asm else frozenset()),)
                elif op.startswith(_LGKM):
                    lgkm = lgkm + ((False, frozenset()),)
                # The hardware counters hold at most 63 vector / 15 LDS operations.
                vm, lgkm = vm[-63:], lgkm[-15:]
                # LDS-queue entries older than its oldest inline-asm read with a destination can
                # neither be reported nor change which of the newer ones a wait retires (a wait
                # keeps the newest N), and no rule reads this queue's length: drop them, so paths
                # that differ only in such entries (the compiler's scalar loads, LDS stores) meet
                # in one state. (The vector queue keeps its length: the wait pairs read it.)
                while lgkm and not lgkm[0][1]:
                    lgkm = lgkm[1:]
                _track_constants(ins, consts)
            pair = _wait_pair(blocks, bi)
            if pair is not None:
                n, flag, join = pair
                waited = n if len(vm) > n else 0
                vm = _retire(vm, waited)
                base = int(re.match(r"s\[(\d+)", flag).group(1))
                consts[base] = -1 if waited else 0
                consts["vcc"] = "zero" if waited else "nonzero"
                items = tuple(sorted(consts.items(), key=lambda kv: str(kv[0])))
                work.append((join, vm, lgkm, items))
                continue
            succs = []
            vcc = consts.get("vcc")
            if block.branch == "s_cbranch_vccnz" and vcc is not None:
                succs = [block.taken] if vcc == "nonzero" else [block.fall]
            elif block.branch == "s_cbranch_vccz" and vcc is not None:
                succs = [block.taken] if vcc == "zero" else [block.fall]
            else:
                succs = [block.fall, block.taken]
            items = tuple(sorted(consts.items(), key=lambda kv: str(kv[0])))
            for succ in succs:
                if succ is not None:
                    work.append((succ, vm, lgkm, items))
        result[name] = [reports[k] for k in sorted(reports)]
    return result
