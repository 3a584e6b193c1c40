"""The CPU attention oracle, pinned (oracle/attention.py).

Against the reference's own golden vectors (tests/golden: the inputs its seeded sample() drew and
its op body's outputs on them, fp64 / fp32 / bf16), against the mathematics (closed forms, an
independent brute-force loop, invariance under a permutation of the pool's pages), and the plan
contract (pad rows zero, the positions assert).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from helpers import digest, golden_args
from workloads import Batch, step_args
from oracle import attention as oracle

DTYPES = {"float64": torch.float64, "float32": torch.float32, "bfloat16": torch.bfloat16}


def _outs(arrays: dict, name: str) -> dict[str, torch.Tensor]:
    out = {}
    for tag in DTYPES:
        key = f"{name}/out_{tag}"
        if key in arrays:
            a = torch.from_numpy(arrays[key])
            out[tag] = a.view(torch.bfloat16) if tag == "bfloat16" else a
    return out


def test_golden_inputs_are_the_reference_draws(golden) -> None:
    """The fixture's inputs, rebuilt at each dtype, are byte for byte the tensors the reference's
    sample() returned at that dtype (sha256 of each, the member's whole arena included)."""
    meta, _ = golden
    for name, entry in meta.items():
        for tag, want in entry["inputs"].items():
            args = golden_args(name, golden, "cpu", DTYPES[tag])
            got = [digest(a) if isinstance(a, torch.Tensor) else a for a in args]
            assert got == want, (name, tag)


def test_oracle_matches_reference_outputs(golden) -> None:
    """The oracle on the reference's inputs reproduces its fp64 truth, its fp32 output, its bf16
    output within bf16 rounding, and its post-append pool bytes."""
    meta, arrays = golden
    for name, entry in meta.items():
        for tag, want in _outs(arrays, name).items():
            args = golden_args(name, golden, "cpu", DTYPES[tag])
            got = oracle.paged_attention(*args)
            if tag == "float64":
                torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-13)
            elif tag == "float32":
                torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-6)
            else:
                # bf16: same fp32 math, rounded once; allow one bf16 ulp where fp32 sums differ
                torch.testing.assert_close(got.float(), want.float(), rtol=2 ** -7, atol=1e-6)
                assert digest(args[3]) == entry["pool_after_bf16"], name


def test_brute_force_agrees_with_oracle(golden) -> None:
    """An independent per-(row, head) Python loop gives the oracle's fp64 result."""
    for name in ("sample_batch", "decode_window", "verify_ragged", "drafter", "prefill_mixed"):
        args = golden_args(name, golden, "cpu", torch.float64)
        want = oracle.paged_attention(*args)
        q, _, _, kv_member, row_request, _, qsl, seq_lens, table, _, window, sinks, causal = args
        got = oracle.brute_force(q, kv_member, row_request, qsl, seq_lens, table, window, sinks,
                                 causal)
        torch.testing.assert_close(got, want, rtol=1e-10, atol=1e-12)


def _single_entry(ctx: int, rows: int, heads=4, kv_heads=2, dim=8, block=4, **kw) -> tuple:
    return step_args(Batch(entries=((ctx, rows),), tokens=rows, reqs=1, heads=heads,
                           kv_heads=kv_heads, head_dim=dim, block=block, **kw), "cpu",
                     torch.float64, seed=3)


def test_one_visible_key_returns_its_value() -> None:
    """Context 0, one row, no sinks: the row sees only its own key, so out = v exactly."""
    args = _single_entry(0, 1, sinks=False)
    out = oracle.paged_attention(*args)
    v = args[2]  # [1, Hkv, D]; q head hq reads kv head hq // G
    want = v.repeat_interleave(2, dim=1).reshape(1, -1)
    torch.testing.assert_close(out, want, rtol=0, atol=1e-15)


def test_equal_keys_give_the_mean_value() -> None:
    """All visible keys equal: uniform weights, out = mean of the visible values."""
    args = list(_single_entry(6, 1, sinks=False))
    kv_member = args[3]
    flat_k, flat_v = oracle.kv_views(kv_member)
    flat_k[:] = 0.5
    args[1] = torch.full_like(args[1], 0.5)  # the appended key equals the cached ones
    out = oracle.paged_attention(*args)
    slots = args[9]
    table = args[8]
    keys = [int(table[0, j // 4]) * 4 + j % 4 for j in range(7)]
    del slots
    mean = flat_v[torch.tensor(keys)].mean(dim=0)  # [Hkv, D] (the appended v was written)
    want = mean.repeat_interleave(2, dim=0).reshape(1, -1)
    torch.testing.assert_close(out, want, rtol=1e-12, atol=1e-12)


def test_sink_with_one_key() -> None:
    """One key with score s and a sink logit z: out = v * e^s / (e^s + e^z)."""
    args = list(_single_entry(0, 1, sinks=True))
    q, k, v = args[0], args[1], args[2]
    sinks = args[11]
    out = oracle.paged_attention(*args)
    for hq in range(4):
        h = hq // 2
        s = float(torch.dot(q[0, hq], k[0, h])) / math.sqrt(8)
        w = math.exp(s) / (math.exp(s) + math.exp(float(sinks[hq])))
        torch.testing.assert_close(out[0, hq * 8:(hq + 1) * 8], v[0, h] * w, rtol=1e-12,
                                   atol=1e-14)


def test_pad_rows_are_zero_and_masked_rows_zero() -> None:
    """Pad rows (row_request -1) are exactly 0, with and without sinks."""
    for sinks in (False, True):
        args = step_args(Batch(entries=((5, 2), (3, 1)), tokens=6, reqs=4, heads=4, kv_heads=2,
                            head_dim=8, block=4, sinks=sinks), "cpu", torch.float32, seed=1)
        out = oracle.paged_attention(*args)
        assert torch.equal(out[3:], torch.zeros_like(out[3:]))
        assert torch.isfinite(out).all()


def test_page_permutation_invariance() -> None:
    """Relabeling the pool's pages (table and pool permuted together) changes nothing."""
    batch = Batch(entries=((21, 3), (9, 1)), tokens=4, reqs=2, heads=4, kv_heads=2, head_dim=8,
                  block=4, window=0, sinks=True)
    args = list(step_args(batch, "cpu", torch.float64, seed=5))
    want = oracle.paged_attention(*[a.clone() if isinstance(a, torch.Tensor) and a.dim() != 5
                                    else a for a in args])
    args = list(step_args(batch, "cpu", torch.float64, seed=5))
    kv_member = args[3]
    pages = kv_member.shape[0]
    perm = torch.cat([torch.zeros(1, dtype=torch.long), torch.randperm(pages - 1) + 1])
    inverse = torch.empty_like(perm)
    inverse[perm] = torch.arange(pages)
    moved = kv_member.clone()
    moved.copy_(kv_member[perm])  # new page i holds old page perm[i]
    # a dense clone is not an arena view; rebuild the member as a view of a fresh arena
    arena = torch.empty(pages, 4, 2, 2, 2, 8, dtype=torch.float64)
    member = arena[:, :, 1].permute(0, 2, 1, 3, 4)
    member.copy_(moved)
    table = inverse[args[8].long()].to(torch.int32)
    slots = args[9]
    new_slots = (inverse[(slots // 4).long()] * 4 + slots % 4).to(torch.int32)
    args[3], args[8], args[9] = member, table, new_slots
    got = oracle.paged_attention(*args)
    torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-14)


def test_positions_assert_refuses_a_bad_plan() -> None:
    args = list(step_args(Batch(entries=((5, 2),), tokens=2, reqs=1, heads=4, kv_heads=2,
                             head_dim=8, block=4), "cpu", torch.float32, seed=0))
    args[5] = args[5].clone()
    args[5][0] += 1
    with pytest.raises(AssertionError):
        oracle.paged_attention(*args)


def test_error_budget_rule() -> None:
    truth = torch.tensor([1.0, -2.0], dtype=torch.float64)
    ref = torch.tensor([1.0, -2.0], dtype=torch.bfloat16)
    assert oracle.error_budget(truth, ref) == pytest.approx(2e-2 * 2.0)
    ref32 = torch.tensor([1.001, -2.0], dtype=torch.float32)
    assert oracle.error_budget(truth, ref32) == pytest.approx(2 * 0.001, rel=1e-3)


def test_chunking_does_not_change_results() -> None:
    """The row-chunk bound is a memory bound only: one-row chunks give the same fp64 result."""
    args = step_args(Batch(entries=((30, 4), (12, 2)), tokens=8, reqs=3, heads=4, kv_heads=2,
                        head_dim=8, block=4, window=5), "cpu", torch.float64, seed=2)
    whole = oracle.paged_attention(*[a.clone() if isinstance(a, torch.Tensor) and a.dim() != 5
                                     else a for a in args])
    args = step_args(Batch(entries=((30, 4), (12, 2)), tokens=8, reqs=3, heads=4, kv_heads=2,
                        head_dim=8, block=4, window=5), "cpu", torch.float64, seed=2)
    tiny = oracle.paged_attention(*args, chunk_bytes=1)
    torch.testing.assert_close(tiny, whole, rtol=1e-13, atol=1e-15)
    assert np.isfinite(tiny.numpy()).all()
