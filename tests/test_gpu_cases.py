"""GPU: the reference's own per-op proof (kelpie/scripts/bench_attention.py), on this build.

Correctness: the 62 cases kelpie grades `paged_attention` on (gpt-oss-20b attention at decode,
prefill, decode_extra and drafter shapes, windows 0 and 128; tests/workloads.reference_cases),
each drawn with seed i by the reference's own generator, graded as the reference grades them
(bench_attention.py:112-140: the fp64 truth, kelpie's error budget, pad rows exactly zero) and by
this build's fixed tolerance (2e-2 + 1e-2 |truth|).

Capture (bench_attention.py:143-185): the reference's two capture shapes -- decode R=8 and a
ragged decode_extra R=4 -- at windows 0 and 128, each captured once in a hipGraph on one plan
and replayed on another of the same shape (the entries reversed: other contexts, rows, pages and
values) written into the captured buffers; a verify-shaped step (1 + 15 causal rows per entry)
and the drafter's non-causal step at the Llama shape; and an fp8 decode step with its fused
quantize-on-append, whose replay must leave the same pool bytes and scales as the eager call.
Every replay equals the eager call on the same inputs, bit for bit.
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


# The reference's capture shapes (bench_attention.py:150-152): (label, entries, tokens, reqs).
CAPTURE_SHAPES = [
    ("decode R=8", [(40, 1), (130, 1), (7, 1), (300, 1), (1, 1), (16, 1), (17, 1), (600, 1)], 8, 8),
    ("decode_extra R=4 ragged", [(40, 16), (130, 3), (7, 1), (300, 9)], 64, 4),
]


@pytest.mark.parametrize("window", [0, 128])
@pytest.mark.parametrize("shape", range(len(CAPTURE_SHAPES)),
                         ids=[label for label, *_ in CAPTURE_SHAPES])
def test_capture_at_the_reference_shapes(shape, window) -> None:
    """gpt-oss attention (64 q / 8 kv heads, D 64, sinks) captured on one plan, replayed three
    times on another of the same shape (the reference's: the entries reversed, so every entry's
    context, rows, pages and values change while the arena and table width stay), with eager
    work in between: each replay equals the eager call, bit for bit, and pad rows stay 0."""
    label, entries, tokens, reqs = CAPTURE_SHAPES[shape]
    say("capture", label, "window", window)

    def batch(e):
        return Batch(entries=tuple(e), tokens=tokens, reqs=reqs, window=window, heads=64,
                     kv_heads=8, head_dim=64, block=16)

    static = list(step_args(batch(entries), "cuda", torch.bfloat16, seed=10))
    fresh = step_args(batch(entries[::-1]), "cuda", torch.bfloat16, seed=11)
    kvpath.paged_attention(*static)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream), torch.cuda.graph(graph, stream=stream):
        out = kvpath.paged_attention(*static)
    torch.cuda.current_stream().wait_stream(stream)
    for dst, src in zip(static, fresh):
        if isinstance(dst, torch.Tensor):
            dst.copy_(src)
    torch.cuda.synchronize()
    n_rows = sum(r for _, r in entries)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        eager = kvpath.paged_attention(*static)
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager), label
        assert not bool(replayed[n_rows:].ne(0).any()), label


def _fp8_decode_step(entries, seed: int):
    batch = Batch(entries=tuple(entries), tokens=len(entries) + 2, reqs=len(entries) + 1,
                  heads=32, kv_heads=8, head_dim=128, block=16, sinks=False)
    return synthetic(batch, "cuda", torch.bfloat16, seed=seed, pool_pages=1024, max_seq_len=8192,
                     cache_dtype=torch.float8_e4m3fn, outliers=0.01)


def test_capture_replays_an_fp8_decode_step() -> None:
    """An fp8 decode step (quantize-on-append fused into the decode kernel) captured on one
    plan and replayed three times on another plan and pool written into the captured buffers:
    each replay's output, pool bytes and scales equal an eager call's from the same starting
    pool, bit for bit. Entries start pages fresh (context a multiple of the page) or append into
    a partly written page, so scales are both set and grown."""
    say("capture fp8 decode")
    first = _fp8_decode_step([(40, 1), (900, 1), (3000, 1), (7, 1), (16, 1), (4095, 1)], 90)
    second = _fp8_decode_step([(2500, 1), (16, 1), (129, 1), (5000, 1), (32, 1), (63, 1)], 91)
    static = list(first.args)
    scale = first.kv_scale
    kvpath.paged_attention_fp8(*static, scale)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream), torch.cuda.graph(graph, stream=stream):
        out = kvpath.paged_attention_fp8(*static, scale)
    torch.cuda.current_stream().wait_stream(stream)
    for dst, src in zip(static, second.args):
        if isinstance(dst, torch.Tensor) and dst is not static[3]:
            dst.copy_(src)
    start_arena, start_scale = second.arena.clone(), second.kv_scale.clone()
    n_rows = second.batch.n_rows
    for _ in range(3):
        first.arena.copy_(start_arena)
        scale.copy_(start_scale)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        replayed, arena_r, scale_r = out.clone(), first.arena.clone(), scale.clone()
        first.arena.copy_(start_arena)
        scale.copy_(start_scale)
        eager = kvpath.paged_attention_fp8(*static, scale)
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager)
        assert not bool(replayed[n_rows:].ne(0).any())
        # Page 0's scratch row takes only the unfused append's pad-row writes; compare the rest.
        assert torch.equal(arena_r[1:].view(torch.uint8), first.arena[1:].view(torch.uint8))
        assert torch.equal(scale_r[1:].view(torch.int32), scale[1:].view(torch.int32))
    assert not torch.equal(scale_r.view(torch.int32), start_scale.view(torch.int32))
