"""Seeded step workloads for the tests and the bench, laid out as kelpie's engine lays them out.

`Batch` describes one layer's step as the reference's generator does (kelpie/kelpie-models/
kelpie_models/kernels/ops/paged_attention.py:270-293). `synthetic` builds it at pool scale (tens of
thousands of pages, millions of context rows) directly on the device: this layer is member m of
an arena of `members` layers (K/V interleaved per row, sdk/kv.py:163-224), pages handed out in a
random order, page 0 the null page, the scratch slot its last row, GARBAGE in never-written
slots, values N(0,1) rounded to bf16. Block tables are as wide as the batch needs, or as wide as
kelpie-core makes them for a `max_seq_len` (scheduler.zig:1577-1578: max_blocks_per_req =
ceil(max_seq_len / block), null pages past each request's own, c_api.zig:1149-1150).
`config_batch` names BASELINE.json's configurations 1-5 and workloads 6-9. Test and bench input
only: the library never imports this module.
"""

from __future__ import annotations

import json
import math
from dataclasses import dataclass, field
from pathlib import Path

import torch

from kvpath.paged_attention import KV_MEMBERS, kv_views, new_kv_scale, no_sinks, write_kv

GARBAGE = 64.0


@dataclass(frozen=True)
class Batch:
    """One layer's step (ops/paged_attention.py:270-293): `entries` is (context already cached,
    rows this step) per real entry; `tokens` / `reqs` the padded T / R (pad rows: entry -1, the
    scratch slot; pad entries: no rows, seq_len 1, an all-null table row)."""

    entries: tuple[tuple[int, int], ...]
    tokens: int
    reqs: int
    heads: int = 64
    kv_heads: int = 8
    head_dim: int = 64
    block: int = 16
    window: int = 0
    sinks: bool = True
    causal: bool = True
    spare_pages: int = 2

    @property
    def n_rows(self) -> int:
        return sum(rows for _, rows in self.entries)


# ---- pool-scale inputs ---------------------------------------------------------------------------


@dataclass
class Step:
    """One generated step: the op's arguments plus what the bench and tests need around them."""

    args: tuple  # the 13 op arguments
    kv_scale: torch.Tensor | None
    batch: Batch
    pool_pages: int
    free_pages: torch.Tensor  # int32 page ids no entry uses (copy_blocks destinations)
    arena: torch.Tensor | None = None  # the whole arena the member views
    extra: dict = field(default_factory=dict)
    member: int = 1  # which of the arena's layers args[3] views

    @property
    def kv_member(self) -> torch.Tensor:
        return self.args[3]


def new_arena(batch: Batch, pool_pages: int, device: str | torch.device, cache_dtype,
              members: int = 2) -> torch.Tensor:
    """An arena of `members` layers over `pool_pages` pages, [pages, block, members, 2, Hkv, D]
    (K/V interleaved per row, every layer's row together, as sdk/kv.py:163-224 lays a group's
    unit out): GARBAGE everywhere, zero bytes for an fp8 cache."""
    b = batch
    shape = (pool_pages, b.block, members, KV_MEMBERS, b.kv_heads, b.head_dim)
    if cache_dtype == torch.float8_e4m3fn:
        return torch.zeros(shape, dtype=torch.uint8, device=device).view(torch.float8_e4m3fn)
    return torch.full(shape, GARBAGE, dtype=cache_dtype, device=device)


def table_width(batch: Batch, max_seq_len: int = 0) -> int:
    """Block-table columns: the batch's widest entry plus spare pages, or kelpie-core's
    max_blocks_per_req = ceil(max_seq_len / block) when `max_seq_len` is given."""
    need = max((-(-(ctx + rows) // batch.block) for ctx, rows in batch.entries), default=1)
    if max_seq_len > 0:
        width = -(-max_seq_len // batch.block)
        assert need <= width, (need, width)
        return width
    return need + batch.spare_pages


def synthetic(batch: Batch, device: str | torch.device, dtype: torch.dtype, seed: int = 0, *,
              pool_pages: int | None = None, outliers: float = 0.0, cache_dtype=None,
              members: int = 2, member: int | None = None, arena: torch.Tensor | None = None,
              max_seq_len: int = 0, chunk_rows: int = 1 << 18) -> Step:
    """`batch` at pool scale, built on the device: this layer is member `member` (default the
    last) of an arena of `members` layers, either a fresh one or `arena` (new_arena) shared with
    other steps, pages drawn at random from its `pool_pages` (the rest stay free), values from a
    device generator. `max_seq_len` > 0 pads every block-table row with null pages to kelpie's
    width for that maximum.

    `outliers` > 0 multiplies that fraction of K/V context elements (and of the step's k/v) by
    20. `cache_dtype=torch.float8_e4m3fn` stores the context through kvpath's quantize-on-append
    (the context is appended as prefill rows in page order, then the step's rows at decode)."""
    b = batch
    device = torch.device(device)
    cache_dtype = dtype if cache_dtype is None else cache_dtype
    gc = torch.Generator(device="cpu").manual_seed(seed)
    gd = torch.Generator(device=device).manual_seed(seed + 1)
    lens = [ctx + rows for ctx, rows in b.entries]
    need = [-(-n // b.block) for n in lens]
    width = table_width(b, max_seq_len)
    used = sum(need)
    if arena is not None:
        pool, members = arena.shape[0], arena.shape[2]
        assert pool >= used + 1, (pool, used)
    else:
        pool = max(pool_pages or 0, used + 1)
        arena = new_arena(b, pool, device, cache_dtype, members)
    member = members - 1 if member is None else member
    perm = (torch.randperm(pool - 1, generator=gc) + 1).to(torch.int32)
    table = torch.zeros(b.reqs, width, dtype=torch.int32)
    at = 0
    for r, n in enumerate(need):
        table[r, :n] = perm[at: at + n]
        at += n
    free_pages = perm[at:].clone()

    kv_member = arena[:, :, member].permute(0, 2, 1, 3, 4)
    kv_scale = new_kv_scale(kv_member) if cache_dtype == torch.float8_e4m3fn else None

    def draw(n: int, heads: int) -> torch.Tensor:
        x = torch.randn(n, heads, b.head_dim, generator=gd, device=device)
        if outliers > 0:
            mask = torch.rand(n, heads, b.head_dim, generator=gd, device=device) < outliers
            x = torch.where(mask, x * 20.0, x)
        return x.to(torch.bfloat16).to(dtype)

    table_dev = table.to(device)
    # Context rows, entry by entry in chunks: slots from the table, values on device.
    for r, (ctx, _) in enumerate(b.entries):
        for c0 in range(0, ctx, chunk_rows):
            n = min(chunk_rows, ctx - c0)
            pos = torch.arange(c0, c0 + n, device=device)
            slots = (table_dev[r, pos // b.block] * b.block + (pos % b.block)).to(torch.int32)
            kc, vc = draw(n, b.kv_heads), draw(n, b.kv_heads)
            if cache_dtype == torch.float8_e4m3fn:
                write_kv(kv_member, kc, vc, slots, kv_scale)
            else:
                flat_k, flat_v = kv_views(kv_member)
                flat_k.index_copy_(0, slots.long(), kc.to(cache_dtype))
                flat_v.index_copy_(0, slots.long(), vc.to(cache_dtype))

    row_request = torch.full((b.tokens,), -1, dtype=torch.int32)
    positions = torch.zeros(b.tokens, dtype=torch.int32)
    slot_mapping = torch.full((b.tokens,), b.block - 1, dtype=torch.int32)
    seq_lens = torch.ones(b.reqs, dtype=torch.int32)
    query_start_loc = torch.full((b.reqs + 1,), b.n_rows, dtype=torch.int32)
    query_start_loc[0] = 0
    row = 0
    for r, (ctx, rows) in enumerate(b.entries):
        pos = torch.arange(ctx, ctx + rows)
        slot_mapping[row: row + rows] = table[r, pos // b.block] * b.block + (pos % b.block).to(
            torch.int32)
        row_request[row: row + rows] = r
        positions[row: row + rows] = pos.to(torch.int32)
        seq_lens[r] = ctx + rows
        row += rows
        query_start_loc[r + 1] = row
    sinks = (torch.randn(b.heads, generator=gc) * 2).to(device) if b.sinks else no_sinks(
        torch.empty(0, device=device))
    q = torch.randn(b.tokens, b.heads, b.head_dim, generator=gd, device=device).to(
        torch.bfloat16).to(dtype)
    k, v = draw(b.tokens, b.kv_heads), draw(b.tokens, b.kv_heads)
    args = (q, k, v, kv_member, row_request.to(device), positions.to(device),
            query_start_loc.to(device), seq_lens.to(device), table_dev, slot_mapping.to(device),
            b.window, sinks, b.causal)
    return Step(args, kv_scale, b, pool, free_pages.to(device), arena, member=member)


def moved(step: Step, device: str | torch.device) -> Step:
    """`step` on `device`: the arena copied whole, the member re-viewed at the same strides."""
    arena = step.arena.to(device)
    kv_member = arena[:, :, step.member].permute(0, 2, 1, 3, 4)
    args = tuple(kv_member if i == 3 else a.to(device) if isinstance(a, torch.Tensor) else a
                 for i, a in enumerate(step.args))
    scale = None if step.kv_scale is None else step.kv_scale.to(device)
    return Step(args, scale, step.batch, step.pool_pages, step.free_pages.to(device), arena,
                dict(step.extra), step.member)


def step_args(batch: Batch, device: str | torch.device, dtype: torch.dtype, seed: int = 0,
              **kw) -> tuple:
    """The op's 13 arguments for a small `batch`, drawn on the CPU by `synthetic` and moved to
    `device`: every device sees the same values, and since each value is drawn in fp32 and
    rounded to bf16 before the cast to `dtype`, the float64 draw of a seed is the bf16 draw's
    exact truth."""
    return moved(synthetic(batch, "cpu", dtype, seed, **kw), device).args


# A small odd case for the op's conventions (ops/paged_attention.py:370-373): GQA 2, one entry
# with context + two rows, one decode row, a pad entry and a pad row, window 3, sinks.
SAMPLE_BATCH = Batch(entries=((5, 2), (3, 1)), tokens=4, reqs=3, heads=4, kv_heads=2,
                     head_dim=32, block=4, window=3)


# ---- the BASELINE configurations -----------------------------------------------------------------

CONFIG_NAMES = {
    1: "tiny_decode_fp32",
    2: "llama3_8b_decode_bf16",
    3: "dflash_verify_bf16",
    4: "fp8_kv_decode",
    5: "long_context_decode_copy_blocks",
    # The callers next to the path (chunked prefill, gpt-oss window + sinks, the DFlash drafter):
    6: "chunked_prefill_bf16",
    7: "gpt_oss_full_decode_bf16",
    8: "gpt_oss_sliding_decode_bf16",
    9: "dflash_drafter_bf16",
    # north_star's own wording of the decode target ("batch 64, ctx 4k"): config 2 at 4096 keys.
    10: "llama3_8b_decode_ctx4k_bf16",
}


def config_batch(cfg: int, seed: int = 0) -> tuple[Batch, dict]:
    """BASELINE.json's configs 1-5, workloads 6-9 of the callers next to the path, and workload
    10 (config 2 with every context at 4096 keys, the decode target's stated shape), as
    (Batch, extras): pool size, dtypes, outliers. Context lengths are drawn from
    `seed` (a CPU generator) as the configs state."""
    g = torch.Generator(device="cpu").manual_seed(1000 + seed)

    def uniform(n: int, lo: int, hi: int) -> list[int]:
        return torch.randint(lo, hi + 1, (n,), generator=g).tolist()

    llama = dict(heads=32, kv_heads=8, head_dim=128, block=16, window=0, sinks=False)
    if cfg == 1:
        lens = [17, 64, 129, 255]  # context including the appended token
        b = Batch(entries=tuple((n - 1, 1) for n in lens), tokens=4, reqs=4, **llama)
        return b, dict(pool_pages=64, dtype=torch.float32)
    if cfg == 2:
        lens = uniform(64, 1024, 4096)
        b = Batch(entries=tuple((n - 1, 1) for n in lens), tokens=64, reqs=64, **llama)
        return b, dict(pool_pages=32768, dtype=torch.bfloat16)
    if cfg == 3:
        ctx = uniform(16, 512, 8192)
        b = Batch(entries=tuple((n, 16) for n in ctx), tokens=256, reqs=16, **llama)
        return b, dict(pool_pages=32768, dtype=torch.bfloat16)
    if cfg == 4:
        lens = uniform(128, 2048, 8192)
        b = Batch(entries=tuple((n - 1, 1) for n in lens), tokens=128, reqs=128, **llama)
        need = sum(math.ceil(n / 16) for n in lens)
        # 4096 free pages beside the context's and the null page (the fp8 append step's pages)
        return b, dict(pool_pages=need + 4096 + 1, dtype=torch.bfloat16,
                       cache_dtype=torch.float8_e4m3fn, outliers=0.01)
    if cfg == 5:
        b = Batch(entries=tuple((131072 - 1, 1) for _ in range(4)), tokens=4, reqs=4,
                  **{**llama, "heads": 64})
        return b, dict(pool_pages=32768 + 4096 + 1, dtype=torch.bfloat16, copy_pairs=4096)
    if cfg == 6:
        # Chunked prefill on the multi-row (MFMA) path: four entries, each a 512-row chunk after
        # 2k cached keys, causal within the chunk (kelpie's prefill bucket family, shapes.py).
        b = Batch(entries=tuple((2048, 512) for _ in range(4)), tokens=2048, reqs=4, **llama)
        return b, dict(pool_pages=32768, dtype=torch.bfloat16)
    gpt_oss = dict(heads=64, kv_heads=8, head_dim=64, block=16, sinks=True)
    if cfg in (7, 8):
        # gpt-oss decode (64 q / 8 kv heads, D 64, per-head sinks, gpt_oss.py:229-249): a full
        # layer (7) and a sliding-window layer, W = 128 (8), at config 2's batch and lengths.
        lens = uniform(64, 1024, 4096)
        b = Batch(entries=tuple((n - 1, 1) for n in lens), tokens=64, reqs=64,
                  window=0 if cfg == 7 else 128, **gpt_oss)
        return b, dict(pool_pages=32768, dtype=torch.bfloat16)
    if cfg == 9:
        # The DFlash drafter's attention (dflash.py:233-320): causal=False over the injected
        # context and the 16-row noise block, config 3's batch and lengths.
        ctx = uniform(16, 512, 8192)
        b = Batch(entries=tuple((n, 16) for n in ctx), tokens=256, reqs=16, causal=False,
                  **{**llama, "sinks": False})
        return b, dict(pool_pages=32768, dtype=torch.bfloat16)
    if cfg == 10:
        # The decode target as north_star words it: batch 64, ctx 4k (4095 cached keys and the
        # appended one), config 2's heads, pages and pool.
        b = Batch(entries=tuple((4095, 1) for _ in range(64)), tokens=64, reqs=64, **llama)
        return b, dict(pool_pages=32768, dtype=torch.bfloat16)
    raise ValueError(f"no config {cfg}")


def copy_pairs(step: Step, n: int, seed: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
    """n (src, dst) page pairs: src among the pages entries use (distinct), dst among the free
    pages (distinct), as config 5's copy_blocks pass draws them."""
    g = torch.Generator(device="cpu").manual_seed(2000 + seed)
    table = step.args[8].cpu()
    live = torch.unique(table[table > 0])
    assert live.numel() >= n and step.free_pages.numel() >= n, (live.numel(), n)
    src = live[torch.randperm(live.numel(), generator=g)[:n]].to(torch.int32)
    free = step.free_pages.cpu()
    dst = free[torch.randperm(free.numel(), generator=g)[:n]].to(torch.int32)
    device = step.kv_member.device
    return src.to(device), dst.to(device)


# ---- the reference's per-op case list --------------------------------------------------------

SHAPES = Path(__file__).resolve().parent / "golden" / "reference_shapes.json"


def _shape_table() -> dict:
    """The reference per-op proof's shape tables, as its own functions returned them
    (tests/golden/make_golden.py writes them from kelpie/scripts/bench_attention.py)."""
    return json.loads(SHAPES.read_text())


def _batch_of(kw: dict, **extra) -> Batch:
    return Batch(**{**kw, "entries": tuple(tuple(e) for e in kw["entries"]), **extra})


def reference_cases() -> list[tuple[str, Batch]]:
    """The 62 shapes kelpie grades `paged_attention` on (kelpie/scripts/bench_attention.py:42-91):
    gpt-oss-20b attention (64 q / 8 kv heads, D 64, block 16, sinks) at the build's step
    families for max_seq_len 512, 8 requests, 1024 batch tokens -- decode R = 1..8 (and 5 real
    entries padded to 8), prefill T = 1..1024 (fresh prompts split over 512-row entries, a chunk
    after 300 cached keys, mixed prefill and decode), decode_extra R x 16 (DFlash's 1 + 15 rows;
    full and ragged) -- each with windows 0 and 128, and the drafter's non-causal, sink-free call
    at the decode_extra shapes. The contexts are the reference's own draws (random.Random(0))."""
    return [(label, _batch_of(kw)) for label, kw in _shape_table()["cases"]]


def reference_buckets() -> list[tuple[str, Batch, bool]]:
    """The reference's timing buckets (bench_attention.py:211-237): its shapes drawn from
    random.Random(1), without the chunked, mixed and 5-real cases, each at windows 0 and 128, as
    (label, batch, graphed): decode-shaped steps are timed as graph replays, prefill eagerly."""
    table = _shape_table()
    out = []
    for label, kw in table["buckets"]:
        for window in (0, 128):
            out.append((f"{label} w{window}", _batch_of(kw, window=window, **table["attention"]),
                        not label.startswith("prefill")))
    return out
