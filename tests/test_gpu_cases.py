"""GPU: the reference's own per-op proof (kelpie/scripts/bench_attention.py), on this build.

Correctness: the 62 cases kelpie grades `paged_attention` on (gpt-oss-20b attention at decode,
prefill, decode_extra and drafter shapes, windows 0 and 128; tests/workloads.reference_cases),
each drawn with seed i by the reference's own generator, graded as the reference grades them
(bench_attention.py:112-140: the fp64 truth, kelpie's error budget, pad rows exactly zero) and by
this build's fixed tolerance (2e-2 + 1e-2 |truth|).

Capture: a verify-shaped step (1 + 15 causal rows per entry) and the drafter's non-causal step,
captured once in a hipGraph; a different plan of the same shape (other contexts, pages, values)
written into the captured buffers; every replay equals the eager call on it
(bench_attention.py:143-185 does the same for its buckets).
"""

from __future__ import annotations

import pytest
import torch

import kvpath
from helpers import within
from oracle import attention as oracle
from test_gpu_path import BF16_ATOL, BF16_RTOL, say
from workloads import Batch, reference_cases, step_args, synthetic

pytestmark = pytest.mark.gpu

CASES = reference_cases()


@pytest.mark.parametrize("index", range(len(CASES)), ids=[label for label, _ in CASES])
def test_reference_case(index) -> None:
    label, batch = CASES[index]
    truth = oracle.paged_attention(*step_args(batch, "cpu", torch.float64, seed=index))
    ref = oracle.paged_attention(*step_args(batch, "cpu", torch.bfloat16, seed=index))
    budget = oracle.error_budget(truth, ref)
    out = kvpath.paged_attention(*step_args(batch, "cuda", torch.bfloat16, seed=index))
    torch.cuda.synchronize()
    got = out.cpu()
    err = (got.double() - truth).abs().max().item()
    pad = got[batch.n_rows:]
    ok, ratio = within(got[:batch.n_rows], truth[:batch.n_rows], BF16_ATOL, BF16_RTOL)
    say(label, "err", f"{err:.3e}", "budget", f"{budget:.3e}", "err/budget",
        round(err / budget, 3), "fixed-tol ratio", round(ratio, 3))
    assert err <= budget, (label, err, budget)
    assert ok, (label, ratio)
    assert not bool(pad.ne(0).any()), label


def _fixed_shape_step(entries, causal: bool, seed: int):
    batch = Batch(entries=tuple(entries), tokens=sum(r for _, r in entries) + 3,
                  reqs=len(entries) + 1, heads=32, kv_heads=8, head_dim=128, block=16,
                  sinks=False, causal=causal)
    # A fixed pool and kelpie-width tables, so two plans of this shape have identical tensors.
    return synthetic(batch, "cuda", torch.bfloat16, seed=seed, pool_pages=1024,
                     max_seq_len=8192)


@pytest.mark.parametrize("causal", [True, False], ids=["verify", "drafter"])
def test_capture_replays_a_new_multi_row_plan(causal) -> None:
    """A verify (causal) or drafter (non-causal) step of 16 rows per entry: capture once, write
    another plan of the same shape into the captured buffers, replay three times with eager work
    in between; each replay equals the eager call, bit for bit, and the pad rows stay zero."""
    say("capture multi-row", "causal" if causal else "non-causal")
    first = _fixed_shape_step([(40, 16), (900, 16), (3000, 16), (7, 16)], causal, 80)
    second = _fixed_shape_step([(2500, 16), (16, 16), (129, 16), (5000, 16)], causal, 81)
    static = list(first.args)
    kvpath.paged_attention(*static)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream), torch.cuda.graph(graph, stream=stream):
        out = kvpath.paged_attention(*static)
    torch.cuda.current_stream().wait_stream(stream)
    first.arena.copy_(second.arena)
    for dst, src in zip(static, second.args):
        if isinstance(dst, torch.Tensor) and dst is not static[3]:
            dst.copy_(src)
    torch.cuda.synchronize()
    n_rows = second.batch.n_rows
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        eager = kvpath.paged_attention(*static)
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager)
        assert not bool(replayed[n_rows:].ne(0).any())
