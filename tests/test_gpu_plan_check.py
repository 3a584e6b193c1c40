"""GPU: the plan check that runs on every op call (kelpie asserts its plan invariant on every
call, kernels/ops/paged_attention.py:128, 143-157).

The kernels derive each row's position from seq_lens and query_start_loc, and a fused append
assumes each new row lands at its position's table slot; the op passes `positions` so the output
writers can check, per row, that the plan is what that derivation assumes. Each case here breaks one thing in an otherwise valid
plan, from the host, with every index still inside the pool and the table, so every kernel runs
to its normal end: the rows that break the plan come back NaN (every head), every other row is
bit-identical to the valid plan's output, and the device's plan-status word is set; the valid
plan leaves it clear. Shapes cover the split-KV path (reduce), one-partition decode and verify
(direct output), prefill, and an fp8 cache.
"""

from __future__ import annotations

import pytest
import torch

import kvpath
from test_gpu_path import say
from workloads import Batch, synthetic

pytestmark = pytest.mark.gpu

LLAMA = dict(heads=32, kv_heads=8, head_dim=128, block=16, sinks=False)
SHAPES = {
    # split-KV decode (reduce writes the rows), the append fused
    "decode_split": (Batch(entries=((3000, 1), (1500, 1), (40, 1), (2047, 1)), tokens=6, reqs=5,
                           **LLAMA), None),
    # decode over a short table: one partition, the decode kernel writes `out`
    "decode_direct": (Batch(entries=((300, 1), (15, 1), (100, 1)), tokens=4, reqs=4, **LLAMA),
                      None),
    # verify: 16 rows per entry, the append fused into the multi-row kernel
    "verify": (Batch(entries=((900, 16), (5000, 16), (31, 16)), tokens=50, reqs=4, **LLAMA), None),
    # gpt-oss verify over a short table: one partition, direct output, sinks
    "verify_direct": (Batch(entries=((200, 16), (40, 7)), tokens=24, reqs=3, heads=64,
                            kv_heads=8, head_dim=64, block=16), None),
    # prefill-sized: separate append launch, then the multi-row kernel
    "prefill": (Batch(entries=((0, 300), (600, 212)), tokens=520, reqs=2, **LLAMA), None),
    # fp8 cache, the quantize-on-append fused into the decode kernel
    "fp8_decode": (Batch(entries=((3000, 1), (1500, 1), (40, 1)), tokens=4, reqs=4, **LLAMA),
                   torch.float8_e4m3fn),
}


def _call(step, args):
    if step.kv_scale is not None:
        return kvpath.paged_attention_fp8(*args, step.kv_scale)
    return kvpath.paged_attention(*args)


def _run(step, args, arena0, scale0):
    """The op on `args` from the step's original pool; -> (out, plan-status bits)."""
    step.arena.copy_(arena0)
    if scale0 is not None:
        step.kv_scale.copy_(scale0)
    kvpath.clear_plan_status()
    out = _call(step, args)
    torch.cuda.synchronize()
    return out.clone(), kvpath.plan_status()


def _nan_rows(out: torch.Tensor) -> set[int]:
    rows = torch.isnan(out.float()).all(dim=1).nonzero().flatten().tolist()
    partial = torch.isnan(out.float()).any(dim=1) & ~torch.isnan(out.float()).all(dim=1)
    assert not bool(partial.any()), "a row is partly NaN"
    return set(rows)


@pytest.mark.parametrize("shape", list(SHAPES))
def test_broken_plans_give_nan_rows_and_set_the_status(shape) -> None:
    batch, cache = SHAPES[shape]
    say("plan check", shape)
    step = synthetic(batch, "cuda", torch.bfloat16, seed=7, pool_pages=2048, cache_dtype=cache)
    args = list(step.args)
    arena0 = step.arena.clone()
    scale0 = step.kv_scale.clone() if step.kv_scale is not None else None
    good, bits = _run(step, args, arena0, scale0)
    assert bits == 0 and not _nan_rows(good), shape
    arena1 = step.arena.clone()  # the pool as the valid call left it: every new row in its slot
    scale1 = step.kv_scale.clone() if step.kv_scale is not None else None
    rr, pos, qsl, lens, table, slots = (args[i] for i in (4, 5, 6, 7, 8, 9))
    qsl_c = qsl.cpu().tolist()
    first = qsl_c[1] - 1  # the last row of entry 0
    fused = shape != "prefill"

    def expect(bad_args: list, broken: set[int], label: str, start=(arena0, scale0)) -> None:
        out, bits = _run(step, bad_args, *start)
        say(" ", label, "status", bits, "NaN rows", sorted(_nan_rows(out)))
        assert bits == 1, label
        assert _nan_rows(out) == broken, label
        keep = torch.ones(out.shape[0], dtype=torch.bool, device=out.device)
        keep[list(broken)] = False
        assert torch.equal(out[keep], good[keep]), label

    # A row one position past its own.
    bad = pos.clone()
    bad[first] += 1
    expect(args[:5] + [bad] + args[6:], {first}, "position off by one")
    # A row naming another entry (inside the plan's entries).
    bad = rr.clone()
    bad[first] = 1
    expect(args[:4] + [bad] + args[5:], {first}, "row_request names another entry")
    # An entry's seq_len past its table row: all of its rows.
    width = table.shape[1]
    bad = lens.clone()
    bad[0] = width * batch.block + 1
    bad_pos = pos.clone()
    n0 = qsl_c[1] - qsl_c[0]
    bad_pos[:n0] = torch.arange(bad[0] - n0, bad[0], dtype=torch.int32, device=pos.device)
    expect(args[:5] + [bad_pos, qsl, bad] + args[8:], set(range(qsl_c[0], qsl_c[1])),
           "seq_len past the table")
    if fused:
        # A fused-append row whose slot is not its position's table slot (a free page's slot,
        # inside the pool): flagged under the opt-in slot check, since the kernels assume the row
        # lands at that table slot; without it the call gives the valid plan's output.
        # Started from the pool the valid call left (the table slot already holds the row, and
        # appending the other rows again writes the same bytes), so the broken row computes what
        # it computed before and only the check tells the calls apart.
        bad = slots.clone()
        free = int(step.free_pages[0])
        bad[first] = free * batch.block + 3
        out, bits = _run(step, args[:9] + [bad] + args[10:], arena1, scale1)
        assert bits == 0 and torch.equal(out, good), "slot check off"
        old = kvpath.set_slot_check(True)
        try:
            expect(args[:9] + [bad] + args[10:], {first}, "slot_mapping off the table",
                   (arena1, scale1))
        finally:
            kvpath.set_slot_check(old)
    kvpath.clear_plan_status()


def test_valid_plans_keep_the_status_clear() -> None:
    """The reference's own case shapes (decode, prefill, decode_extra, drafter; padded plans
    among them) leave the plan-status word clear, with the slot check on."""
    from workloads import reference_cases

    kvpath.clear_plan_status()
    old = kvpath.set_slot_check(True)
    try:
        for i, (label, batch) in enumerate(reference_cases()[::5]):
            step = synthetic(batch, "cuda", torch.bfloat16, seed=i)
            kvpath.paged_attention(*step.args)
    finally:
        kvpath.set_slot_check(old)
    assert kvpath.plan_status() == 0


def test_plan_lengths_are_refused_before_any_launch() -> None:
    """The C++ ops check the plan's lengths on the host: a plan tensor shorter or longer than the
    contract's raises ValueError naming it, and nothing is launched (the cache and the status
    word are untouched)."""
    batch, _ = SHAPES["decode_split"]
    step = synthetic(batch, "cuda", torch.bfloat16, seed=7, pool_pages=2048)
    args = list(step.args)
    arena0 = step.arena.clone()
    kvpath.clear_plan_status()
    rr, pos, qsl, lens, table, slots = (args[i] for i in (4, 5, 6, 7, 8, 9))
    cases = {
        "row_request": (4, rr[:-1]),
        "positions": (5, torch.cat([pos, pos[:1]])),
        "query_start_loc": (6, qsl[:-1]),
        "block_table": (8, table[:-1]),
        "slot_mapping": (9, slots[:-1]),
    }
    for what, (i, bad) in cases.items():
        say("plan length", what, tuple(bad.shape))
        with pytest.raises(ValueError, match=what):
            kvpath.paged_attention(*(args[:i] + [bad] + args[i + 1:]))
    with pytest.raises(ValueError, match="slot_mapping"):
        kvpath.write_kv(step.kv_member, args[1], args[2], slots[:-1])
    torch.cuda.synchronize()
    assert torch.equal(step.arena, arena0)
    assert kvpath.plan_status() == 0
