"""GPU: the path shards over kv heads with no exchange.

Tensor parallelism over attention heads (gpt-oss shards them so, models/torch/gpt_oss.py:99-146)
gives each rank Hkv/tp kv heads of every page and the matching q heads; block tables, slot
mapping and the rest of the plan are replicated. The kernels take the member's strides and head
counts as parameters, so a rank runs the same op on its head slice of the cache view. Here the
ranks run one after another on one GPU, over head slices of the same pool: with the partition
length fixed, the concatenated outputs equal the unsharded call's bit for bit and the pool ends
byte for byte the same past the null page (each head's work is independent of the others');
under the library's own split, whose slot count follows the step's workgroup count (R x Hkv),
each rank may split long entries differently, so the outputs agree within the bf16 tolerance.
"""

from __future__ import annotations

import pytest
import torch

import kvpath
from test_gpu_path import BF16_ATOL, BF16_RTOL, say
from workloads import Batch, synthetic

pytestmark = pytest.mark.gpu

LLAMA = dict(heads=32, kv_heads=8, head_dim=128, block=16)
SHAPES = {
    "decode": Batch(entries=((3000, 1), (1500, 1), (40, 1), (2047, 1)), tokens=6, reqs=5, **LLAMA),
    "verify": Batch(entries=((900, 16), (5000, 16), (31, 16)), tokens=50, reqs=4, **LLAMA),
    "prefill": Batch(entries=((0, 300), (600, 212)), tokens=520, reqs=2, **LLAMA),
    "gpt_oss_window": Batch(entries=((700, 1), (300, 1), (2000, 1)), tokens=4, reqs=4, heads=64,
                            kv_heads=8, head_dim=64, block=16, window=128, sinks=True),
}


def _shards(args: list, tp: int, partition: int) -> torch.Tensor:
    """The op rank by rank over head slices of the same views; -> [T, H * D] concatenated."""
    q, k, v, member, sinks = args[0], args[1], args[2], args[3], args[11]
    n_tok, heads, dim = q.shape
    kv_heads = member.shape[3]
    outs = []
    for rank in range(tp):
        h0, h1 = rank * kv_heads // tp, (rank + 1) * kv_heads // tp
        g0, g1 = h0 * heads // kv_heads, h1 * heads // kv_heads
        sargs = list(args)
        sargs[0], sargs[1], sargs[2] = q[:, g0:g1], k[:, h0:h1], v[:, h0:h1]
        sargs[3] = member[:, :, :, h0:h1]
        sargs[11] = sinks[g0:g1] if sinks.numel() else sinks
        outs.append(kvpath.paged_attention(*sargs, partition=partition).view(n_tok, g1 - g0, dim))
    torch.cuda.synchronize()
    return torch.cat(outs, dim=1).view(n_tok, heads * dim)


@pytest.mark.parametrize("tp", [2, 4])
@pytest.mark.parametrize("shape", list(SHAPES))
def test_head_shards_equal_the_whole_call(shape, tp) -> None:
    batch = SHAPES[shape]
    say("shards", shape, "tp", tp)
    step = synthetic(batch, "cuda", torch.bfloat16, seed=5, pool_pages=1024)
    args = list(step.args)
    arena0 = step.arena.clone()
    for partition in (256, 0):
        step.arena.copy_(arena0)
        whole = kvpath.paged_attention(*args, partition=partition)
        torch.cuda.synchronize()
        whole, arena_whole = whole.clone(), step.arena.clone()
        step.arena.copy_(arena0)
        sharded = _shards(args, tp, partition)
        # Pages past the null one: pad rows append to page 0's scratch slot, all of them to the
        # same one, so its bytes are whichever write lands last (nothing reads it).
        assert torch.equal(step.arena[1:], arena_whole[1:]), (shape, tp, partition)
        if partition:
            assert torch.equal(sharded, whole), (shape, tp)
        else:
            err = (sharded.float() - whole.float()).abs()
            bound = BF16_ATOL + BF16_RTOL * whole.float().abs()
            assert bool((err <= bound).all()), (shape, tp, err.max().item())
