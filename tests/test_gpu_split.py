"""GPU: the split-KV partitioning is decided per sequence on the device, so it does not depend on
how wide kelpie makes the block table (kelpie-core/src/scheduler.zig:1577-1578 sizes it for
max_seq_len, c_api.zig:1149-1150 pads it with null pages).

The same step at the batch's own width and at kelpie's widths for max_seq_len 8k and 128k must
give the same output bit for bit (same partitions, same arithmetic), and match the fp64 oracle;
config 5's 128k contexts in 256 fixed partitions of 512 keys (BASELINE config 5 as stated) and
in the library's own split agree with each other and with the oracle.
"""

from __future__ import annotations

import pytest
import torch

import kvpath
from test_gpu_path import BF16_ATOL, BF16_RTOL, FP8_ATOL, FP8_RTOL, _check_against_oracle, say
from workloads import Batch, config_batch, synthetic

pytestmark = pytest.mark.gpu


def _run(step) -> torch.Tensor:
    if step.kv_scale is not None:
        out = kvpath.paged_attention_fp8(*step.args, step.kv_scale)
    else:
        out = kvpath.paged_attention(*step.args)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("cfg", [2, 3, 4, 9])
def test_kelpie_table_width_gives_the_same_output(cfg) -> None:
    """Configs 2 (decode), 3 (verify), 4 (fp8 decode) and 9 (drafter) at the batch's own table
    width and at kelpie's widths for max_seq_len 8k and 128k: the split and every output bit are
    the same, and the output matches the fp64 oracle."""
    batch, extra = config_batch(cfg)
    outs = {}
    for msl in (0, 8192, 131072):
        say("config", cfg, "max_seq_len", msl)
        step = synthetic(batch, "cuda", extra["dtype"], seed=cfg, pool_pages=extra["pool_pages"],
                         outliers=extra.get("outliers", 0.0), cache_dtype=extra.get("cache_dtype"),
                         max_seq_len=msl)
        width = step.args[8].shape[1]
        split = kvpath.split_plan(batch.tokens, batch.reqs, batch.heads, batch.kv_heads, width,
                                  batch.block)
        say("  table width", width, "split", split)
        outs[msl] = (_run(step).cpu(), split)
        if msl == 131072:
            subset = {2: [0, 17, 63], 3: [0, 15], 4: [0, 127], 9: [0, 15]}[cfg]
            atol, rtol = (FP8_ATOL, FP8_RTOL) if step.kv_scale is not None else (BF16_ATOL, BF16_RTOL)
            _check_against_oracle(outs[msl][0].cuda(), step.args, subset, atol, rtol,
                                  step.kv_scale, f"config {cfg} at 128k width")
        del step
    for msl in (8192, 131072):
        assert outs[msl][1] == outs[0][1], (msl, outs[msl][1], outs[0][1])
        assert torch.equal(outs[msl][0], outs[0][0]), msl


def test_config5_in_256_partitions() -> None:
    """BASELINE config 5 as stated: 128k contexts split into 256 partitions of 512 keys (the
    general reduce over 256 partials per row), against the fp64 oracle and against the library's
    own split (65 slots of 2048 keys) within fp32/bf16 rounding of the partials."""
    batch, extra = config_batch(5)
    step = synthetic(batch, "cuda", extra["dtype"], seed=5, pool_pages=extra["pool_pages"])
    q, k, v, kv_member, rr, pos, qsl, lens, table, slots, window, sinks, causal = step.args
    kvpath.write_kv(kv_member, k, v, slots)
    width = table.shape[1]
    part, n_slots, per_entry = kvpath.split_plan(batch.tokens, batch.reqs, batch.heads,
                                                 batch.kv_heads, width, batch.block, 512)
    assert (part, per_entry) == (512, False) and n_slots >= 256, (part, n_slots)
    fixed = kvpath.attend(q, kv_member, rr, qsl, lens, table, window, sinks, causal, partition=512)
    own = kvpath.attend(q, kv_member, rr, qsl, lens, table, window, sinks, causal)
    torch.cuda.synchronize()
    say("config 5: 512-key partitions", n_slots, "slots; library split",
        kvpath.split_plan(batch.tokens, batch.reqs, batch.heads, batch.kv_heads, width, batch.block))
    torch.testing.assert_close(fixed.float(), own.float(), atol=4e-3, rtol=8e-3)
    _check_against_oracle(fixed, step.args, [0, 3], BF16_ATOL, BF16_RTOL, None,
                          "config 5, 256 partitions")


def test_split_invariance_at_kelpie_width() -> None:
    """At kelpie's 128k width, fixed partitions of 96, 512 and 4096 keys and the library's own
    per-sequence split agree within fp32/bf16 rounding (decode and verify rows, a window)."""
    for rows, window in ((1, 0), (16, 0), (1, 300)):
        batch = Batch(entries=((900, rows), (3000, rows), (17, rows), (6000, rows)),
                      tokens=4 * rows, reqs=4, heads=32, kv_heads=8, head_dim=128, block=16,
                      window=window, sinks=True)
        step = synthetic(batch, "cuda", torch.bfloat16, seed=rows + window, pool_pages=2048,
                         max_seq_len=131072)
        q, k, v, kv_member, rr, pos, qsl, lens, table, slots, w, sinks, causal = step.args
        kvpath.write_kv(kv_member, k, v, slots)
        outs = [kvpath.attend(q, kv_member, rr, qsl, lens, table, w, sinks, causal,
                              partition=p).float() for p in (0, 96, 512, 4096)]
        say("split invariance rows", rows, "window", window)
        for o in outs[1:]:
            torch.testing.assert_close(o, outs[0], atol=4e-3, rtol=8e-3)
        _check_against_oracle(outs[0].to(torch.bfloat16), step.args, None, BF16_ATOL, BF16_RTOL,
                              None, f"kelpie width rows {rows} window {window}")
