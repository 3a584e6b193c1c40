"""The attention kernels' inline-asm loads against the compiler's register allocation (CPU).

Untracked loads need the compiler to leave each destination register alone until the explicit
wait; the scan (kvpath.isa_scan, run by kvpath.build.build() before it links) checks the gfx950
assembly, built with the library's own flags, for any copy or reuse before that wait. (At D 256
the bf16 decode kernel once copied its K registers into AGPRs right after the loads and reused
them for an address: a GPU memory fault whenever the data landed in between.)
"""

from __future__ import annotations

import shutil
from pathlib import Path

import pytest

from kvpath import build
from kvpath.isa_scan import scan

SRC = build.CSRC / "attention.hip"
HAVE_HIPCC = shutil.which("hipcc") is not None or Path("/opt/rocm/bin/hipcc").exists()


def test_scanner_flags_a_copy_before_the_wait() -> None:
    """The scan itself: a copy of an inline-asm load's destination before its wait is reported;
    the same copy after the wait is not, nor are the compiler's own loads."""
    bad = """_Zkernel: ; @k
\t;;#ASMSTART
\tglobal_load_dwordx4 v[6:9], v[34:35], off
\t;;#ASMEND
\tv_accvgpr_write_b32 a150, v6
\ts_waitcnt vmcnt(0)
\ts_endpgm
"""
    good = bad.replace("\tv_accvgpr_write_b32 a150, v6\n\ts_waitcnt vmcnt(0)\n",
                       "\ts_waitcnt vmcnt(0)\n\tv_accvgpr_write_b32 a150, v6\n")
    tracked = bad.replace("\t;;#ASMSTART\n", "").replace("\t;;#ASMEND\n", "")
    assert scan(bad)["_Zkernel"]
    assert not scan(good)["_Zkernel"]
    assert not scan(tracked)["_Zkernel"]
    # A counted wait retires all but the newest loads.
    two = """_Zkernel: ; @k
\t;;#ASMSTART
\tglobal_load_dwordx4 v[6:9], v[34:35], off
\t;;#ASMEND
\t;;#ASMSTART
\tglobal_load_dwordx4 v[10:13], v[36:37], off
\t;;#ASMEND
\ts_waitcnt vmcnt(1)
\tv_mov_b32_e32 v0, v6
\tv_mov_b32_e32 v1, v10
\ts_endpgm
"""
    reports = scan(two)["_Zkernel"]
    assert len(reports) == 1 and "v1, v10" in reports[0]


# A loop whose body ends by issuing the next iteration's load and branches back to a header that
# copies the destination before waiting: reached only along the back-edge.
BACK_EDGE = """_Zkernel: ; @k
\ts_waitcnt vmcnt(0)
.LBB0_1:                                ; =>This Loop Header: Depth=1
\tv_accvgpr_write_b32 a150, v6
\ts_waitcnt vmcnt(0)
\tv_mov_b32_e32 v0, v6
\t;;#ASMSTART
\tglobal_load_dwordx4 v[6:9], v[34:35], off
\t;;#ASMEND
\ts_cmp_lt_i32 s2, s3
\ts_cbranch_scc1 .LBB0_1
; %bb.2:
\ts_waitcnt vmcnt(0)
\ts_endpgm
"""


def _linear_scan(asm: str) -> list[str]:
    """The scan as it was before it followed the control-flow graph: program order, pending
    loads kept across conditional branches and dropped at an unconditional one."""
    import re

    from kvpath.isa_scan import _regs, _retire

    vm, reports, in_asm = [], [], False
    for line in asm.split("\n")[1:]:
        s = line.strip()
        if s.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if s.startswith(";;#ASMEND"):
            in_asm = False
            continue
        if not s or s.startswith((";", ".")) or s.endswith(":"):
            continue
        op = s.split()[0]
        if op == "s_waitcnt":
            vm = list(_retire(tuple(vm), int(re.search(r"vmcnt\((\d+)\)", s).group(1))))
            continue
        if op in ("s_branch", "s_endpgm"):
            vm = []
            continue
        if op.startswith("s_cbranch"):
            continue
        operands = s[len(op):]
        live = set().union(*[r for a, r in vm if a]) if vm else set()
        if _regs(operands) & live:
            reports.append(s)
        if op.startswith("global_load"):
            vm.append((in_asm, _regs(operands.split(",")[0])))
    return reports


def test_scanner_follows_loop_back_edges() -> None:
    """A load outstanding at a loop's back-edge is outstanding at its header: reported. The
    program-order scan this replaces walked past it (the header comes before the load)."""
    assert not _linear_scan(BACK_EDGE)
    reports = scan(BACK_EDGE)["_Zkernel"]
    assert len(reports) == 1 and "a150, v6" in reports[0]
    fixed = BACK_EDGE.replace("\tv_accvgpr_write_b32 a150, v6\n\ts_waitcnt vmcnt(0)\n",
                              "\ts_waitcnt vmcnt(0)\n\tv_accvgpr_write_b32 a150, v6\n")
    assert not scan(fixed)["_Zkernel"]


# The compiled form of `load(block 0); if (two) load(block 1); if (two) wait(1); else wait(0);
# use(block 0)`: the wait pair holds its choice in s[0:1] (set to -1, cleared where it waits for
# everything) and tests it with s_andn2_b64 vcc / s_cbranch_vccnz around the counted wait.
WAIT_PAIR = """_Zkernel: ; @k
\t;;#ASMSTART
\tglobal_load_dwordx4 v[6:9], v[34:35], off
\t;;#ASMEND
\ts_cmp_lt_i32 s4, 2
\ts_cbranch_scc1 .LBB0_2
; %bb.1:
\t;;#ASMSTART
\tglobal_load_dwordx4 v[10:13], v[36:37], off
\t;;#ASMEND
.LBB0_2:
\ts_cmp_ge_i32 s5, s4
\ts_mov_b64 s[0:1], -1
\ts_cbranch_scc0 .LBB0_4
; %bb.3:
\t;;#ASMSTART
\ts_waitcnt vmcnt(0)
\t;;#ASMEND
\ts_mov_b64 s[0:1], 0
.LBB0_4:
\ts_andn2_b64 vcc, exec, s[0:1]
\ts_cbranch_vccnz .LBB0_6
; %bb.5:
\t;;#ASMSTART
\ts_waitcnt vmcnt(1)
\t;;#ASMEND
.LBB0_6:
\tv_mov_b32_e32 v0, v6
\ts_waitcnt vmcnt(0)
\tv_mov_b32_e32 v1, v10
\ts_endpgm
"""


def test_scanner_takes_a_wait_pair_as_one_wait() -> None:
    """A compiled if/else pair of waits is one wait: wait(1) with a second block in flight,
    wait(0) without. No path through it leaves block 0 outstanding, so using block 0 after it is
    clean; using it before the pair is reported, and so is a look-alike whose second branch tests
    another flag (not a pair: the path that skips both waits is real there)."""
    assert not scan(WAIT_PAIR)["_Zkernel"]
    early = WAIT_PAIR.replace(".LBB0_2:\n", ".LBB0_2:\n\tv_mov_b32_e32 v2, v7\n")
    assert any("v2, v7" in r for r in scan(early)["_Zkernel"])
    other_flag = WAIT_PAIR.replace("s_andn2_b64 vcc, exec, s[0:1]", "s_andn2_b64 vcc, exec, s[2:3]")
    assert any("v0, v6" in r for r in scan(other_flag)["_Zkernel"])


def test_scanner_merges_paths_that_differ_in_register_less_lds_entries(monkeypatch) -> None:
    """The LDS queue's entries older than its oldest inline-asm read carry nothing to report and
    cannot change which reads a wait retires, so the scan drops them: a read behind a scalar load
    and an LDS store is still reported when used early; a register-less entry issued after the
    read still counts for lgkmcnt(N); and paths that differ only in such entries meet in one
    state (a chain of twelve optional scalar loads scans within 100 block visits, where keeping
    every queue length apart takes several hundred)."""
    early = """_Zkernel: ; @k
\ts_load_dword s0, s[2:3], 0x0
\tds_write_b32 v1, v2
\t;;#ASMSTART
\tds_read_b128 v[6:9], v10
\t;;#ASMEND
\tv_mov_b32_e32 v0, v6
\ts_waitcnt lgkmcnt(0)
\ts_endpgm
"""
    reports = scan(early)["_Zkernel"]
    assert len(reports) == 1 and "v0, v6" in reports[0]
    newer = """_Zkernel: ; @k
\t;;#ASMSTART
\tds_read_b128 v[6:9], v10
\t;;#ASMEND
\tds_write_b32 v1, v2
\ts_waitcnt lgkmcnt(1)
\tv_mov_b32_e32 v0, v6
\ts_endpgm
"""
    assert not scan(newer)["_Zkernel"]
    assert scan(newer.replace("lgkmcnt(1)", "lgkmcnt(2)"))["_Zkernel"]
    chain = ["_Zkernel: ; @k"]
    for i in range(12):
        chain += [f"\ts_cmp_lt_i32 s4, {i}", f"\ts_cbranch_scc1 .LBB0_{i}",
                  f"; %bb.x{i}:", f"\ts_load_dword s{10 + i}, s[2:3], 0x{4 * i:x}", f".LBB0_{i}:"]
    chain += ["\t;;#ASMSTART", "\tds_read_b128 v[6:9], v10", "\t;;#ASMEND", "\ts_waitcnt lgkmcnt(0)",
              "\tv_mov_b32_e32 v0, v6", "\ts_endpgm", ""]
    monkeypatch.setattr("kvpath.isa_scan._MAX_VISITS", 100)
    assert not scan("\n".join(chain))["_Zkernel"]


def test_build_refuses_a_hazard() -> None:
    """kvpath.build.build() scans the assembly before linking: a report raises."""
    build.refuse_hazards({"clean.s": BACK_EDGE.replace(
        "\tv_accvgpr_write_b32 a150, v6\n\ts_waitcnt vmcnt(0)\n",
        "\ts_waitcnt vmcnt(0)\n\tv_accvgpr_write_b32 a150, v6\n")})
    with pytest.raises(build.IsaHazardError, match="a150, v6"):
        build.refuse_hazards({"loop.s": BACK_EDGE})


@pytest.mark.skipif(not HAVE_HIPCC, reason="hipcc is not installed")
def test_attention_kernels_keep_async_destinations(tmp_path) -> None:
    """Every kernel of attention.hip: no instruction touches a register that an outstanding
    inline-asm load will still write, on any path of the control-flow graph."""
    out = build.assemble(SRC, tmp_path / "attention.s")
    reports = scan(out.read_text())
    kernels = [k for k in reports if "attn_" in k]
    assert len(kernels) >= 20, kernels
    bad = {k: v[:3] for k, v in reports.items() if v}
    assert not bad, bad
