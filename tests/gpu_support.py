"""Helpers for the GPU parity tests: move a step to the CPU in a compact form the oracle can run,
and select a subset of a plan's entries."""

from __future__ import annotations

import torch

from kvpath.paged_attention import KV_MEMBERS
from workloads import GARBAGE


def compact_cpu(args: tuple, entries: list[int] | None = None, kv_scale=None) -> tuple:
    """The op arguments restricted to `entries` (default: all), on the CPU, with only the pages
    those entries use copied into a fresh arena (page 0 = null page) and the table, slot mapping
    renumbered. Values are bit-identical; the oracle on the result equals the oracle on the
    original for the kept rows. Returns (args_cpu, rows kept (index tensor into T), scale_cpu)."""
    (q, k, v, kv_member, row_request, positions, qsl, seq_lens, table, slot_mapping, window,
     sinks, causal) = args
    R = seq_lens.shape[0]
    entries = list(range(R)) if entries is None else list(entries)
    qsl_c, lens_c, table_c = qsl.cpu(), seq_lens.cpu(), table.cpu()
    block = kv_member.shape[2]
    keep_rows, new_qsl, new_lens, new_rr = [], [0], [], []
    used_pages = [0]
    for i, r in enumerate(entries):
        a, b = int(qsl_c[r]), int(qsl_c[r + 1])
        keep_rows.extend(range(a, b))
        new_rr.extend([i] * (b - a))
        new_qsl.append(new_qsl[-1] + (b - a))
        new_lens.append(int(lens_c[r]))
        n = -(-int(lens_c[r]) // block)
        used_pages.extend(int(p) for p in table_c[r, :n])
    pages = torch.tensor(sorted(set(used_pages)), dtype=torch.long)
    remap = {int(p): i for i, p in enumerate(pages)}
    width = max(1, max(-(-n // block) for n in new_lens)) if new_lens else 1
    new_table = torch.zeros(len(entries), width, dtype=torch.int32)
    for i, r in enumerate(entries):
        n = -(-new_lens[i] // block)
        new_table[i, :n] = torch.tensor([remap[int(p)] for p in table_c[r, :n]], dtype=torch.int32)
    heads, dim = kv_member.shape[3], kv_member.shape[4]
    fp8 = kv_member.dtype == torch.float8_e4m3fn
    raw = kv_member.view(torch.uint8) if fp8 else kv_member  # index fp8 pages as bytes
    dev_pages = raw[pages.to(kv_member.device)]  # [n, 2, block, Hkv, D] dense copy
    arena = torch.full((pages.numel(), block, 1, KV_MEMBERS, heads, dim),
                       0 if fp8 else GARBAGE, dtype=raw.dtype)
    member = arena[:, :, 0].permute(0, 2, 1, 3, 4)
    member.copy_(dev_pages.cpu())
    if fp8:
        member = member.view(torch.float8_e4m3fn)
    rows = torch.tensor(keep_rows, dtype=torch.long)
    slots_c = slot_mapping.cpu()[rows]
    new_slots = torch.tensor([remap[int(s) // block] * block + int(s) % block for s in slots_c],
                             dtype=torch.int32)
    scale_c = kv_scale[pages.to(kv_scale.device)].cpu().contiguous() if kv_scale is not None else None
    out = (q.cpu()[rows], k.cpu()[rows], v.cpu()[rows], member,
           torch.tensor(new_rr, dtype=torch.int32), positions.cpu()[rows],
           torch.tensor(new_qsl, dtype=torch.int32), torch.tensor(new_lens, dtype=torch.int32),
           new_table, new_slots, window, sinks.cpu(), causal)
    return out, rows, scale_c


def dequantized(member_fp8: torch.Tensor, scale: torch.Tensor,
                dtype: torch.dtype = torch.float64) -> torch.Tensor:
    """An fp8 member (CPU) as values e4m3 * scale[page, member, head] in `dtype`, in an
    arena-layout view (K/V interleaved per row) so the oracle's kv_views can flatten it. The
    product is formed in f64, where it is exact (4 + 24 significant bits), so an f32 result is
    the f32 product rounded once, as an f32 dequantize computes it."""
    vals = member_fp8.to(torch.float32).to(torch.float64)
    vals = (vals * scale.to(torch.float64)[:, :, None, :, None]).to(dtype)
    pages, _, block, heads, dim = vals.shape
    arena = torch.empty(pages, block, 1, KV_MEMBERS, heads, dim, dtype=dtype)
    member = arena[:, :, 0].permute(0, 2, 1, 3, 4)
    member.copy_(vals)
    return member
