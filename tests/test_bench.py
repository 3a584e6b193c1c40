"""bench.py's contract on the CPU: the multi-GPU refusal, and the algorithmic byte count that the
roofline's `achieved` divides by the kernel's time, against closed forms on small batches."""

from __future__ import annotations

import json
import math
import subprocess
import sys

import bench
from workloads import Batch


def _decode(lens, heads=32, kv_heads=8, dim=128, window=0):
    return Batch(entries=tuple((n - 1, 1) for n in lens), tokens=len(lens), reqs=len(lens),
                 heads=heads, kv_heads=kv_heads, head_dim=dim, block=16, window=window)


def test_multi_gpu_refused() -> None:
    """`--gpus 2` prints one JSON line naming the reason and exits 2, before touching a GPU."""
    proc = subprocess.run([sys.executable, str(bench.ROOT / "bench.py"), "--gpus", "2"],
                          capture_output=True, text=True, timeout=120)
    assert proc.returncode == 2
    line = json.loads(proc.stdout.strip().splitlines()[-1])
    assert "one GPU" in line["error"]


def test_decode_bytes_closed_form() -> None:
    """Decode rows see every key of their entry: K and V once per key and kv head, q and out
    once, one table entry per page, and one partial (D bf16 + two f32) per row, q head and
    partition the entry's keys touch."""
    lens = [100, 513, 1024]
    b = bench.step_bytes(_decode(lens), kv_itemsize=2, q_itemsize=2, partition=512)
    hkv, d, h = 8, 128, 32
    kv = sum(lens) * 2 * hkv * d * 2
    assert b["kv"] == kv
    parts = sum(h * math.ceil(n / 512) for n in lens) * (d * 2 + 8)
    q = out = len(lens) * h * d * 2
    table = sum(math.ceil(n / 16) for n in lens) * 4
    assert b["partition"] == kv + q + table + parts
    assert b["reduce"] == parts + out
    assert b["append"] == len(lens) * (2 * hkv * d * (2 + 2) + 4)
    assert b["flops"] == sum(h * n * 4 * d for n in lens)


def test_f32_partials_and_direct_output() -> None:
    """f32 partials count 4 bytes a value; a direct-output step has no partials or reduce."""
    lens = [300, 700]
    f32 = bench.step_bytes(_decode(lens), partition=512, part_itemsize=4)
    bf16 = bench.step_bytes(_decode(lens), partition=512, part_itemsize=2)
    n_partials = sum(32 * math.ceil(n / 512) for n in lens)
    assert f32["reduce"] - bf16["reduce"] == n_partials * 128 * 2
    direct = bench.step_bytes(_decode(lens), partition=1024, direct=True)
    assert direct["reduce"] == 0
    assert direct["partition"] == direct["kv"] + 2 * len(lens) * 32 * 128 * 2 + \
        sum(math.ceil(n / 16) for n in lens) * 4


def test_window_and_fp8_bytes() -> None:
    """A sliding window reads only the keys it shows (from the first visible key's page on for
    the table); an fp8 cache reads 1 byte a value plus two f32 scales per page and kv head."""
    b = bench.step_bytes(_decode([1000], window=128), partition=512)
    assert b["kv"] == 128 * 2 * 8 * 128 * 2
    fp8 = bench.step_bytes(_decode([1000]), kv_itemsize=1, partition=512)
    pages = math.ceil(1000 / 16)
    assert fp8["kv"] == 1000 * 2 * 8 * 128 + pages * 2 * 8 * 4


def test_verify_rows_are_causal() -> None:
    """Multi-row (verify) entries: row i of r rows sits at n - r + i and sees keys up to itself;
    the entry's K/V is counted once, its flops per row."""
    batch = Batch(entries=((84, 16),), tokens=16, reqs=1, heads=32, kv_heads=8, head_dim=128,
                  block=16)
    b = bench.step_bytes(batch, partition=512)
    assert b["kv"] == 100 * 2 * 8 * 128 * 2
    assert b["flops"] == sum(32 * (84 + i + 1) * 4 * 128 for i in range(16))


def test_per_entry_split_covers_each_entry() -> None:
    """The library's per-entry split (mirrored in bench.entry_split): partitions of a multiple of
    32 keys, at most `slots` of them, at most the floor length while the slots suffice, covering
    [anchor, n) with no partition left empty; a window anchors at the first visible key's
    32-key block."""
    for n in (1, 31, 32, 33, 511, 512, 513, 1500, 4096, 4097, 8208, 131072):
        for slots in (1, 3, 9, 65):
            anchor, part = bench.entry_split(n, 1, 0, 512, slots)
            count = -(-(n - anchor) // part)
            assert anchor == 0 and part % 32 == 0 and 1 <= count <= slots, (n, slots, part)
            if -(-n // 512) <= slots:
                assert part <= 512 and count == -(-n // 512), (n, slots, part)
            assert (count - 1) * part < n - anchor <= count * part
    anchor, part = bench.entry_split(1000, 1, 128, 512, 9, 1)
    assert anchor == (1000 - 1 - 128 + 1) // 32 * 32 and part >= 1000 - anchor
    assert bench.entry_split(1000, 1, 0, 384, None) == (0, 384)


def test_split_bytes_count_partitions_per_entry() -> None:
    """With the per-entry split, each decode row writes one partial per partition of its own
    entry: ceil(n / 512) while that fits the slots, else `slots`."""
    lens = [100, 1500, 4096, 6000]
    b = bench.step_bytes(_decode(lens), partition=512, slots=9)
    counts = [min(9, -(-n // 512)) for n in lens]
    parts = sum(32 * c for c in counts) * (128 * 2 + 8)
    assert b["reduce"] == parts + len(lens) * 32 * 128 * 2


def test_published_buckets_are_timed() -> None:
    """Every bucket the reference publishes microseconds for (kelpie/NOTES-attn.md:44-49) is one
    `bench.py --cases` times, at the reference's shapes: decode R=1 is one row over one entry,
    decode_extra R=8 is 8 entries of 16 rows, the prefills are fresh prompts of 128 and 1024
    rows in 512-row entries; decode-shaped buckets are graph replays, prefill eager."""
    from workloads import reference_buckets

    buckets = {label: (batch, graphed) for label, batch, graphed in reference_buckets()}
    assert len(buckets) == 46
    assert set(bench.PUBLISHED_US) <= set(buckets)
    batch, graphed = buckets["decode R=1 w0"]
    assert (batch.n_rows, len(batch.entries), graphed) == (1, 1, True)
    batch, graphed = buckets["decode_extra R=8 w0"]
    assert [rows for _, rows in batch.entries] == [16] * 8 and graphed
    batch, graphed = buckets["prefill T=1024 fresh w0"]
    assert batch.entries == ((0, 512), (0, 512)) and not graphed
    batch, _ = buckets["decode R=8 w128"]
    assert batch.window == 128 and (batch.heads, batch.kv_heads, batch.head_dim) == (64, 8, 64)
