"""The reference's own input generator, restated for the tests: `sample(batch, device, dtype,
seed)` returns, draw for draw, the tensors kelpie's `sample()` returns (kelpie/kelpie-models/
kelpie_models/kernels/ops/paged_attention.py:270-373): K/V interleaved per row of a two-member
page (`kv_member` is a strided view, like the arena's), pages handed out in a random order, page
0 the null page, the scratch slot its last row, GARBAGE in never-written slots, values drawn in
fp32 and rounded to bf16 so a float64 sample is the bf16 sample's exact truth. The golden
fixtures (tests/golden) pin it byte for byte. Test input only: the library never imports it.
"""

from __future__ import annotations

import torch

from kvpath.paged_attention import KV_MEMBERS, kv_views, no_sinks
from workloads import GARBAGE, Batch


def sample(batch: Batch, device: str | torch.device, dtype: torch.dtype, seed: int = 0) -> tuple:
    """The op's 13 arguments for `batch` (ops/paged_attention.py:300-367, same draw order)."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    b = batch
    assert b.n_rows <= b.tokens and len(b.entries) <= b.reqs, b
    assert b.heads % b.kv_heads == 0, b

    def draw(*shape: int) -> torch.Tensor:
        return torch.randn(*shape, generator=g).to(torch.bfloat16).to(device=device, dtype=dtype)

    lens = [ctx + rows for ctx, rows in b.entries]
    need = [-(-n // b.block) for n in lens]
    width = max(need, default=1) + b.spare_pages
    n_pages = 1 + sum(need)
    order = (torch.randperm(n_pages - 1, generator=g) + 1).tolist()
    table = torch.zeros(b.reqs, width, dtype=torch.int32)
    for r, n in enumerate(need):
        table[r, :n] = torch.tensor(order[:n], dtype=torch.int32)
        order = order[n:]
    arena = torch.full((n_pages, b.block, 2, KV_MEMBERS, b.kv_heads, b.head_dim), GARBAGE,
                       dtype=dtype, device=device)
    kv_member = arena[:, :, 1].permute(0, 2, 1, 3, 4)
    flat_k, flat_v = kv_views(kv_member)
    flat_k[: b.block].copy_(draw(b.block, b.kv_heads, b.head_dim))
    flat_v[: b.block].copy_(draw(b.block, b.kv_heads, b.head_dim))

    row_request = torch.full((b.tokens,), -1, dtype=torch.int32)
    positions = torch.zeros(b.tokens, dtype=torch.int32)
    slot_mapping = torch.full((b.tokens,), b.block - 1, dtype=torch.int32)
    seq_lens = torch.ones(b.reqs, dtype=torch.int32)
    query_start_loc = torch.full((b.reqs + 1,), b.n_rows, dtype=torch.int32)
    query_start_loc[0] = 0
    row = 0
    for r, (ctx, rows) in enumerate(b.entries):
        pos = torch.arange(ctx + rows)
        slots = table[r, pos // b.block] * b.block + (pos % b.block).to(torch.int32)
        flat_k.index_copy_(0, slots[:ctx].to(device).long(), draw(ctx, b.kv_heads, b.head_dim))
        flat_v.index_copy_(0, slots[:ctx].to(device).long(), draw(ctx, b.kv_heads, b.head_dim))
        row_request[row: row + rows] = r
        positions[row: row + rows] = torch.arange(ctx, ctx + rows, dtype=torch.int32)
        slot_mapping[row: row + rows] = slots[ctx:]
        seq_lens[r] = ctx + rows
        row += rows
        query_start_loc[r + 1] = row
    sinks = (torch.randn(b.heads, generator=g) * 2).to(device) if b.sinks else no_sinks(
        torch.empty(0, device=device))
    return (
        draw(b.tokens, b.heads, b.head_dim),
        draw(b.tokens, b.kv_heads, b.head_dim),
        draw(b.tokens, b.kv_heads, b.head_dim),
        kv_member,
        row_request.to(device),
        positions.to(device),
        query_start_loc.to(device),
        seq_lens.to(device),
        table.to(device),
        slot_mapping.to(device),
        b.window,
        sinks,
        b.causal,
    )


# A small odd case, the reference's own (ops/paged_attention.py:370-373): GQA 2, one entry with
# context + two rows, one decode row, a pad entry and a pad row, window 3, sinks.
SAMPLE_BATCH = Batch(entries=((5, 2), (3, 1)), tokens=4, reqs=3, heads=4, kv_heads=2,
                     head_dim=32, block=4, window=3)
