#!/usr/bin/env python3
"""Benchmark of Kelpie's paged-KV hot path on one MI355X: one step = the whole op at BASELINE
config 2 (Llama-3-8B-shape decode: batch 64, context U[1k, 4k] seeded, 32 q / 8 kv heads, D 128,
block 16, bf16, a 32k-page pool): append 1 token per sequence at its slot, then split-KV paged
attention (each sequence split by its own length, <= 512-key partitions at this shape) and the
reduce. The default run also measures every other config at its full shape in the same process
(`also`: configs 3-5, workloads 6-9, and workload 10: config 2 with every context at 4096 keys,
the decode target's stated "batch 64, ctx 4k"), the KV append at a bandwidth-sized step (bf16, and fp8
whole pages) and config 5's copy_blocks.
`--config N` measures BASELINE config N (1-5) or workload N (6-9: chunked prefill, gpt-oss full
and sliding-window decode, the DFlash drafter; 10: config 2 at 4096 keys) alone.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--config 2] [--partition 0]
                    [--max-seq-len 0] [--members 2]

Prints ONE JSON line. `value` = algorithmic HBM bytes of the step / its time (GB/s); the step
is captured in a hipGraph of K back-to-back steps (the way kelpie serves decode, sdk/captured.py),
inputs resident in HBM, rotating over three independent pools (3 x 0.65 GB of KV) so the 256 MB
Infinity Cache cannot serve a repeat. `roofline` is for the dominant kernel (the partition
kernel), timed alone the same way (K launches in one hipGraph, HIP events on the stream it
replays on); above the bf16 ridge (prefill) it is in TFLOP/s against the MFMA peak.
`cpu_baseline` times the reference algorithm's CPU restatement (oracle/) on the same step shape
on this host's cores.

`--max-seq-len` pads every block table to kelpie's width for that maximum (kelpie-core sizes
tables for max_seq_len, scheduler.zig:1577-1578); `--members N` makes this layer one of N in the
arena's unit (sdk/kv.py:202-222: at N = 32, Llama-3-8B's 32 layers, rows of 128 KiB and pages of
2 MiB), the three rotations then being three layers of one arena.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path[:0] = [str(ROOT), str(ROOT / "research-2_amd"), str(ROOT / "tests")]

HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E, 8 TB/s
MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, 2.5 PFLOP/s
CONFIG = 2
ALSO = (10, 3, 4, 5, 6, 7, 8, 9)  # measured beside the headline in the default run (10 first: the
# decode target's other reading, taken right after config 2)
ROTATE = 3
APPEND_ROWS = 65536
METRIC = "paged decode attn HBM GB/s (% peak) + tokens/s; KV append GB/s; 1 MI355X"


def log(*parts) -> None:
    print("[bench]", *parts, file=sys.stderr, flush=True)


def entry_split(n: int, rows: int, window: int, partition: int, slots: int | None,
                grid_slots: int | None = None) -> tuple[int, int]:
    """(anchor, partition length) of an entry of n keys whose last `rows` are this step's, as the
    library splits it: a fixed `partition` when `slots` is None, else its own split of the keys
    from the anchor into min(grid slots, ceil(span / partition)) partitions of equal length
    rounded up to 32 keys (attention.hip split_entry)."""
    anchor = max(0, n - rows - window + 1) // 32 * 32 if window > 0 else 0
    if slots is None:
        return anchor, partition
    span = n - anchor
    count = min(max(-(-span // partition), 1), grid_slots or slots)
    return anchor, -(-(-(-span // count)) // 32) * 32


def step_bytes(batch, kv_itemsize: int = 2, q_itemsize: int = 2, partition: int = 512,
               direct: bool = False, part_itemsize: int = 2,
               slots: int | None = None) -> dict[str, int]:
    """Algorithmic bytes of one step, per kernel. KV read = every key some row of an entry can
    see, K and V once (2 * Hkv * D * kv_itemsize per key), plus for an fp8 cache the two f32
    scales per (page, kv head); a row of entry (n keys, r rows) at i sits at position
    n - r + i and sees keys [pos - window + 1, pos] (causal) or [.., n) (not causal).
    Partials = per (row, q head, partition its keys span) D values of `part_itemsize` bytes
    (bf16 for a bf16 q, else f32) and two f32, written by the partition kernel and read by the
    reduce; partitions are `partition` keys each, or with `slots` each entry's own split
    (entry_split). Append = each new row read (q dtype) and written (cache dtype) once, plus its
    slot. `direct`: the partition kernel writes the output itself (one partition per entry), so
    there are no partials and no reduce."""
    hkv, d, h, block = batch.kv_heads, batch.head_dim, batch.heads, batch.block
    window, causal = batch.window, batch.causal
    grid_slots = slots
    if slots is not None and window > 0:
        grid_slots = min(slots, -(-(window + batch.tokens + 30) // partition))
    kv = table = parts = flops = 0
    for ctx, rows in batch.entries:
        n = ctx + rows
        anchor, part = entry_split(n, rows, window, partition, slots, grid_slots)
        spans = []
        for i in range(rows):
            pos = n - rows + i
            hi = pos + 1 if causal else n
            lo = max(0, pos - window + 1) if window > 0 else 0
            spans.append((lo, hi))
            flops += h * (hi - lo) * 4 * d  # q.k and p.v, 2 * D each per (row, head, key)
            n_parts = (hi - 1 - anchor) // part - (lo - anchor) // part + 1
            parts += h * n_parts * (d * part_itemsize + 8)
        lo, hi = min(a for a, _ in spans), max(b for _, b in spans)
        kv += (hi - lo) * 2 * hkv * d * kv_itemsize
        n_pages = math.ceil(hi / block) - lo // block
        table += n_pages * 4
        if kv_itemsize == 1:
            kv += n_pages * 2 * hkv * 4
    q = batch.tokens * h * d * q_itemsize
    out = batch.tokens * h * d * q_itemsize
    append = batch.tokens * (2 * hkv * d * (q_itemsize + kv_itemsize) + 4)
    if direct:
        return {"append": append, "partition": kv + q + table + out, "reduce": 0, "kv": kv,
                "flops": flops}
    return {"append": append, "partition": kv + q + table + parts, "reduce": parts + out,
            "kv": kv, "flops": flops}


def time_graph(fn, rotations: list, steps: int, warmup: int) -> float:
    """ms per step of fn(rotation): `warmup` steps, then exactly `steps` steps, each set captured
    as ONE hipGraph of back-to-back steps rotating over the pools (as kelpie captures a whole
    decode step, sdk/captured.py) and replayed once; HIP events on the current stream bracket
    the timed replay, synchronized around."""
    import torch

    def capture(n: int):
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream), torch.cuda.graph(g, stream=stream):
            for i in range(n):
                fn(rotations[i % len(rotations)])
        torch.cuda.current_stream().wait_stream(stream)
        return g

    for rot in rotations:  # eager once per rotation (lazy init, allocator warm)
        fn(rot)
    torch.cuda.synchronize()
    warm = capture(max(warmup, 1))
    timed = capture(steps)
    torch.cuda.synchronize()
    warm.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    timed.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


# The reference's published microseconds per layer for its buckets (kelpie/NOTES-attn.md:44-49:
# gpt-oss attention, decode-shaped steps as graph replays, prefill eager), on A100 and H100, for
# its reference op and for vLLM's Triton kernel. Context beside the figures measured here, not a
# target. Keys are this bench's bucket labels (NOTES: "decode_extra R=8 x16 w0" is the full
# decode_extra R=8 bucket, "prefill T=128 w0" the fresh prefill).
PUBLISHED_US = {
    "decode R=1 w0": {"A100 ref": 79.9, "A100 vllm": 24.6, "H100 ref": 63.1, "H100 vllm": 19.8},
    "decode R=8 w0": {"A100 ref": 209.9, "A100 vllm": 34.8, "H100 ref": 148.7, "H100 vllm": 25.5},
    "decode R=8 w128": {"A100 ref": 215.0, "A100 vllm": 22.5, "H100 ref": 153.5, "H100 vllm": 18.1},
    "decode_extra R=8 w0": {"A100 ref": 1946.6, "A100 vllm": 51.2, "H100 ref": 1259.2,
                            "H100 vllm": 35.2},
    "prefill T=128 fresh w0": {"A100 ref": 1031, "A100 vllm": 250, "H100 ref": 738,
                               "H100 vllm": 158},
    "prefill T=1024 fresh w0": {"A100 ref": 13451, "A100 vllm": 360, "H100 ref": 8998,
                                "H100 vllm": 232},
}
CASE_REPLAYS = 50
CASE_WARMUP = 5
CASE_LAYERS = 24  # gpt-oss-20b's attention layers


def time_call(fn, args: tuple, graphed: bool, calls: int = 1) -> float:
    """Median microseconds of one call over CASE_REPLAYS, as the reference times its buckets
    (bench_attention.py:189-208): one call captured in a hipGraph and replayed, HIP events around
    each replay; or, eagerly, HIP events around each call. With `calls` > 1 (graphed only) the
    graph holds that many back-to-back calls, as a captured model step holds one per layer, and
    each replay's time is divided by it."""
    import torch

    fn(*args)
    torch.cuda.synchronize()
    if graphed:
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream), torch.cuda.graph(graph, stream=stream):
            for _ in range(calls):
                fn(*args)
        torch.cuda.current_stream().wait_stream(stream)
        run = graph.replay
    else:
        def run() -> None:
            fn(*args)
    for _ in range(CASE_WARMUP):
        run()
    times = []
    for _ in range(CASE_REPLAYS):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        run()
        end.record()
        end.synchronize()
        times.append(start.elapsed_time(end) * 1e3 / calls)
    return statistics.median(times)


def reference_buckets_line() -> dict:
    """Microseconds per layer for the reference's timing buckets (workloads.reference_buckets),
    each drawn on the device by workloads.synthetic with seed 20, the published A100 / H100
    figures beside the six buckets kelpie/NOTES-attn.md lists."""
    import torch

    import kvpath
    from kvpath import _lib
    from workloads import reference_buckets, synthetic

    _lib.load()  # fails loudly without the HIP library
    rows = []
    for label, batch, graphed in reference_buckets():
        args = synthetic(batch, "cuda", torch.bfloat16, seed=20).args
        us = time_call(kvpath.paged_attention, args, graphed)
        row = {"bucket": label, "us_per_layer": round(us, 2), "timing": "graph" if graphed else "eager",
               "rows": batch.n_rows, "tokens": batch.tokens}
        if graphed:
            # The same call once per layer of a captured step (gpt-oss-20b's 24 layers, no other
            # ops between them): the per-layer cost without a graph launch per call.
            row["us_per_layer_in_step"] = round(time_call(kvpath.paged_attention, args, True,
                                                          CASE_LAYERS), 2)
        if label in PUBLISHED_US:
            row["published_us"] = PUBLISHED_US[label]
        rows.append(row)
        log(f"{label}: {us:.2f} us ({row['timing']})"
            + (f", {row['us_per_layer_in_step']:.2f} us in a {CASE_LAYERS}-layer graph" if graphed else ""))
        del args
        torch.cuda.empty_cache()
    return {"mode": "reference_buckets", "unit": "us per layer (gpt-oss attention: 64 q / 8 kv "
            "heads, D 64, block 16, sinks; append + attention, one op call; us_per_layer_in_step: "
            f"one call per layer of a {CASE_LAYERS}-call graph)", "n_gpus": 1,
            "published": "kelpie/NOTES-attn.md:44-49 (A100/H100; context, not a target)",
            "rows": rows, "memory": peak_memory_rows()}


# The reference's memory shapes (bench_attention.py:244-245): its largest prefill, two ways.
MEMORY_SHAPES = (("prefill T=1024 2x512", ((0, 512), (0, 512)), 1024, 2),
                 ("prefill T=1024 1x1024", ((0, 1024),), 1024, 1))


def peak_memory_rows() -> list[dict]:
    """Peak device memory one eager op call allocates above its inputs, as the reference
    measures it (bench_attention.py:241-261): torch's allocator peak after a reset, minus what
    was allocated before the call. The op's output and its split-KV workspace are all it
    allocates."""
    import torch

    import kvpath
    from workloads import Batch, synthetic

    rows = []
    for label, entries, tokens, reqs in MEMORY_SHAPES:
        batch = Batch(entries=entries, tokens=tokens, reqs=reqs, window=0, heads=64, kv_heads=8,
                      head_dim=64, block=16)
        args = synthetic(batch, "cuda", torch.bfloat16, seed=0).args
        torch.cuda.synchronize()
        base = torch.cuda.memory_allocated()
        torch.cuda.reset_peak_memory_stats()
        out = kvpath.paged_attention(*args)
        torch.cuda.synchronize()
        peak = torch.cuda.max_memory_allocated() - base
        rows.append({"shape": label, "peak_bytes_above_inputs": int(peak),
                     "peak_gib": round(peak / 2**30, 6), "output_bytes": out.numel() * 2})
        log(f"memory {label}: {peak / 2**20:.2f} MiB above inputs (output "
            f"{out.numel() * 2 / 2**20:.2f} MiB)")
        del args, out
        torch.cuda.empty_cache()
    return rows


def measured_traffic(kernel: str, workload: str) -> int | None:
    """HBM bytes per launch of `kernel` on `workload` from the committed rocprofv3 counter
    summary (FETCH_SIZE scaled by its copy-kernel calibration, plus WRITE_SIZE), or None when
    no summary covers this kernel and workload."""
    for path in sorted((ROOT / "profiles").glob("traffic_*.json")):
        rec = json.loads(path.read_text())
        if rec.get("kernel") == kernel and rec.get("workload") == workload:
            return int(rec["traffic_bytes_per_launch"])
    return None


def cpu_baseline(batch, cfg: int, total_bytes: int) -> dict:
    """The reference algorithm's CPU restatement (oracle.attention: index_copy_ append, chunked
    gather over the batch's occupied width, fp32 GQA einsum, masked softmax) on the whole step of
    config `cfg`, on this host's cores: warmup 3, median of 10 (kelpie bench/timing.py:17-36);
    GB/s over the same algorithmic bytes as the GPU line."""
    import torch

    from oracle import attention as oracle
    from workloads import synthetic

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    args = synthetic(batch, "cpu", torch.bfloat16, seed=0).args
    for _ in range(3):
        oracle.paged_attention(*args)
    times = []
    for _ in range(10):
        t0 = time.perf_counter()
        oracle.paged_attention(*args)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    return {"value": round(total_bytes / t / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"the whole config-{cfg} step ({len(batch.entries)} entries, append + "
                      f"attention), bf16 inputs, fp32 compute; median of 10 after 3 warmups; "
                      f"{t * 1e3:.1f} ms per step",
            "ms_per_step": round(t * 1e3, 3)}


def kernel_name(batch, dtype, fp8: bool, direct: bool) -> str:
    """The partition kernel the library launches for this step (its rocprofv3 name)."""
    import torch

    g_heads = batch.heads // batch.kv_heads
    multi_row = batch.tokens > len(batch.entries)
    # Row tiles per wave: two for bf16 steps of 16+ tiles per entry at D <= 128, else one.
    tiles = math.ceil(math.ceil(batch.tokens * g_heads / batch.reqs) / 16)
    tpw = 2 if tiles >= 16 and batch.head_dim <= 128 else 1
    flag = "true" if fp8 else "false"
    if dtype == torch.float32:
        return "attn_partition_generic"
    if multi_row and fp8:
        return f"attn_partition_mfma<{batch.head_dim},{flag}>"
    if multi_row:
        return f"attn_partition_verify<{batch.head_dim},{tpw},4>"
    return f"attn_partition_mfma_decode<{batch.head_dim},{flag},{str(direct).lower()}>"


def measure(cfg: int, args, *, extras: bool) -> dict:
    """Time config `cfg`'s step and its partition kernel; with `extras`, also the side
    measurements the config carries (append at bandwidth size, copy_blocks)."""
    import ctypes

    import torch

    import kvpath
    from kvpath import _lib
    from kvpath.paged_attention import _cache, _dtype_code, _opts, _plan, _rows, _stream, _workspace
    from workloads import CONFIG_NAMES, config_batch, copy_pairs, new_arena, synthetic

    lib = _lib.load()  # fails loudly without the HIP library
    batch, extra = config_batch(cfg)
    dtype, cache_dtype = extra["dtype"], extra.get("cache_dtype")
    fp8 = cache_dtype == torch.float8_e4m3fn
    log("building", ROTATE, "pools for config", cfg)
    shared = None
    if args.members >= ROTATE:  # the rotations are three layers of one arena
        shared = new_arena(batch, extra["pool_pages"], "cuda", cache_dtype or dtype, args.members)
    rots = [synthetic(batch, "cuda", dtype, seed=s, pool_pages=extra["pool_pages"],
                      outliers=extra.get("outliers", 0.0), cache_dtype=cache_dtype,
                      members=args.members, arena=shared,
                      member=s if shared is not None else None, max_seq_len=args.max_seq_len)
            for s in range(ROTATE)]
    torch.cuda.synchronize()

    width = rots[0].args[8].shape[1]
    part, slots, per_entry = kvpath.split_plan(batch.tokens, batch.reqs, batch.heads,
                                               batch.kv_heads, width, batch.block, args.partition)

    def op(st) -> None:
        if st.kv_scale is not None:
            kvpath.paged_attention_fp8(*st.args, st.kv_scale, partition=args.partition)
        else:
            kvpath.paged_attention(*st.args, partition=args.partition)

    # The step: the whole op.
    ms_step = time_graph(op, rots, args.steps, args.warmup)
    log(f"config {cfg} step {ms_step * 1e3:.1f} us")

    # The dominant kernel alone: the split-KV partition pass over the appended pools. The
    # library's rule for direct output: when the grid holds one partition per entry (a short
    # table, or a window that fits a partition), the decode kernel (bf16 or fp8 cache) or the
    # bf16 multi-row kernel normalizes and writes `out` itself; kvpath_attend then launches that
    # kernel alone, so it is what is timed.
    g_heads = batch.heads // batch.kv_heads
    multi_tile = math.ceil(math.ceil(batch.tokens * g_heads / batch.reqs) / 16) > 1
    grid_slots = (min(slots, math.ceil((batch.window + batch.tokens + 30) / part))
                  if batch.window > 0 else slots)
    direct = grid_slots == 1 and dtype == torch.bfloat16 and (not multi_tile or not fp8)
    part_state = []
    for st in rots:
        q, k, v, kv_member, rr, pos, qsl, lens, table, slot_map, window, sinks, causal = st.args
        cache = _cache(kv_member, st.kv_scale)
        qr, qq = _rows(q, "q")
        plan, keep = _plan(rr, qsl, lens, table, slot_map, q.shape[0])
        opts, sinks_f32 = _opts(window, sinks, q.shape[1], causal, args.partition)
        ws = _workspace(q.device, q.shape[0], lens.shape[0], q.shape[1], kv_member.shape[3],
                        q.shape[2], table.shape[1], kv_member.shape[2], args.partition)
        out = torch.empty(q.shape[0], q.shape[1] * q.shape[2], dtype=q.dtype, device=q.device)
        outr = _lib.Rows(out.data_ptr(), q.shape[0], q.shape[1], q.shape[2], out.stride(0),
                         q.shape[2], _dtype_code(out, "out"))
        part_state.append((cache, qr, qq, plan, keep, opts, ws, sinks_f32, out, outr))

    def partitions(state) -> None:
        cache, qr, _, plan, _, opts, ws, _, _, outr = state
        stream = _stream(torch.device("cuda", 0))
        if direct:
            _lib.check("attend", lib.kvpath_attend(
                ctypes.byref(qr), ctypes.byref(cache), ctypes.byref(plan), ctypes.byref(opts),
                ctypes.byref(outr), ws.data_ptr(), ws.numel(), stream))
        else:
            _lib.check("attend_partitions", lib.kvpath_attend_partitions(
                ctypes.byref(qr), ctypes.byref(cache), ctypes.byref(plan), ctypes.byref(opts),
                ws.data_ptr(), ws.numel(), stream))

    # K launches of the kernel alone captured in one hipGraph, as the step is: back-to-back on
    # the GPU with no host launch cost between them (which would dominate a 10 us kernel).
    ms_part = time_graph(partitions, part_state, max(args.steps, 30), args.warmup)
    log(f"config {cfg} partition kernel {ms_part * 1e3:.1f} us")

    kv_item = 1 if fp8 else (4 if dtype == torch.float32 else 2)
    q_item = 4 if dtype == torch.float32 else 2
    # The library keeps split-KV partials in bf16 for a bf16 q, in f32 otherwise.
    part_item = 2 if dtype == torch.bfloat16 else 4
    b = step_bytes(batch, kv_item, q_item, part, direct, part_item,
                   slots if per_entry else None)
    total = b["append"] + b["partition"] + b["reduce"]
    value = total / (ms_step * 1e-3) / 1e9
    part_gbps = b["partition"] / (ms_part * 1e-3) / 1e9
    kernel = kernel_name(batch, dtype, fp8, direct)
    workload = CONFIG_NAMES[cfg]
    res = {
        "workload": workload,
        "config": {"workload": workload, "batch": len(batch.entries),
                   "rows_per_entry": batch.entries[0][1], "q_heads": batch.heads,
                   "kv_heads": batch.kv_heads, "head_dim": batch.head_dim,
                   "block_size": batch.block, "pool_pages": extra["pool_pages"],
                   "table_width": width, "members": args.members,
                   "window": batch.window, "sinks": batch.sinks, "causal": batch.causal,
                   "split": {"partition_tokens": part, "slots": slots, "per_entry": per_entry},
                   "step": ("append + attention (one partition per entry, output written "
                            "directly)" if direct else "append + split-KV attention + reduce"),
                   "timing": "K steps captured in one hipGraph, replayed once"},
        "dtype": "fp8_e4m3 kv / bf16" if fp8 else str(dtype).removeprefix("torch."),
        "pool_pages": extra["pool_pages"],
        "value": value,
        "ms_per_step": ms_step,
        "pct_peak_hbm": round(100 * value / HBM_PEAK_GBPS, 1),
        "tokens_per_s": round(batch.n_rows / (ms_step * 1e-3), 1),
        "tokens_per_s_32_layers": round(batch.n_rows / (32 * ms_step * 1e-3), 1),
        "step_bytes": total,
        "roofline": {"kernel": kernel, "bound": "hbm",
                     "achieved": round(part_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(part_gbps / HBM_PEAK_GBPS, 4),
                     "traffic": measured_traffic(kernel, workload),
                     "us_per_launch": round(ms_part * 1e3, 2),
                     "algorithmic_bytes": b["partition"]},
        "batch": batch,
    }
    # Above the ridge (peak flops / peak bytes) the partition kernel is bounded by MFMA rate.
    if b["flops"] / b["partition"] > MFMA_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBPS * 1e9):
        tflops = b["flops"] / (ms_part * 1e-3) / 1e12
        res["roofline"].update({"bound": "mfma", "achieved": round(tflops, 1),
                                "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                                "frac": round(tflops / MFMA_PEAK_TFLOPS, 4),
                                "algorithmic_flops": b["flops"]})

    if extras and cfg == 2:
        # KV append at a bandwidth-sized step: 65,536 rows into the pool, distinct slots.
        g = torch.Generator().manual_seed(9)
        app = []
        for st in rots:
            pool_slots = st.kv_member.shape[0] * batch.block
            slot_t = (torch.randperm(pool_slots - batch.block, generator=g)[:APPEND_ROWS]
                      + batch.block).to(torch.int32).cuda()
            kk = torch.randn(APPEND_ROWS, batch.kv_heads, batch.head_dim, device="cuda").to(dtype)
            vv = torch.randn(APPEND_ROWS, batch.kv_heads, batch.head_dim, device="cuda").to(dtype)
            app.append((st.kv_member, kk, vv, slot_t))
        ms_app = time_graph(lambda a: kvpath.write_kv(*a), app, args.steps, args.warmup)
        app_bytes = APPEND_ROWS * (2 * batch.kv_heads * batch.head_dim * 2 * 2 + 4)
        log(f"append {APPEND_ROWS} rows {ms_app * 1e3:.1f} us")
        res["kv_append"] = {
            "rows": APPEND_ROWS, "us": round(ms_app * 1e3, 2),
            "GBps": round(app_bytes / (ms_app * 1e-3) / 1e9, 1),
            "pct_peak_hbm": round(100 * app_bytes / (ms_app * 1e-3) / 1e9 / HBM_PEAK_GBPS, 1)}
    if extras and fp8:
        # fp8 quantize-on-append at a bandwidth-sized step: 65,536 rows as 4096 whole pages
        # (prefill-shaped: each page written from its row 0, so it starts afresh), free pages.
        n_pages = APPEND_ROWS // batch.block
        g = torch.Generator().manual_seed(10)
        app = []
        for st in rots:
            free = st.free_pages.cpu()
            assert free.numel() >= n_pages, (free.numel(), n_pages)
            pages = free[torch.randperm(free.numel(), generator=g)[:n_pages]].to(torch.int64)
            slot_t = (pages[:, None] * batch.block + torch.arange(batch.block)).reshape(-1)
            kk = torch.randn(APPEND_ROWS, batch.kv_heads, batch.head_dim, device="cuda").to(dtype)
            vv = torch.randn(APPEND_ROWS, batch.kv_heads, batch.head_dim, device="cuda").to(dtype)
            app.append((st.kv_member, kk, vv, slot_t.to(torch.int32).cuda(), st.kv_scale))
        ms_app = time_graph(lambda a: kvpath.write_kv(*a), app, args.steps, args.warmup)
        app_bytes = (APPEND_ROWS * (2 * batch.kv_heads * batch.head_dim * (2 + 1) + 4)
                     + n_pages * 2 * batch.kv_heads * 4)
        log(f"fp8 append {APPEND_ROWS} rows {ms_app * 1e3:.1f} us")
        res["kv_append_fp8"] = {
            "rows": APPEND_ROWS, "pages": n_pages, "us": round(ms_app * 1e3, 2),
            "GBps": round(app_bytes / (ms_app * 1e-3) / 1e9, 1),
            "pct_peak_hbm": round(100 * app_bytes / (ms_app * 1e-3) / 1e9 / HBM_PEAK_GBPS, 1)}
    if extras and "copy_pairs" in extra:
        pairs = [copy_pairs(st, extra["copy_pairs"], seed=i) for i, st in enumerate(rots)]
        args_copy = [(st.kv_member, src, dst) for st, (src, dst) in zip(rots, pairs)]
        ms_copy = time_graph(lambda a: kvpath.copy_blocks(*a), args_copy, args.steps, args.warmup)
        page_bytes = 2 * batch.block * batch.kv_heads * batch.head_dim * kv_item
        copy_bytes = 2 * extra["copy_pairs"] * page_bytes
        log(f"copy_blocks {extra['copy_pairs']} pairs {ms_copy * 1e3:.1f} us")
        res["copy_blocks"] = {
            "pairs": extra["copy_pairs"], "us": round(ms_copy * 1e3, 2),
            "GBps": round(copy_bytes / (ms_copy * 1e-3) / 1e9, 1),
            "pct_peak_hbm": round(100 * copy_bytes / (ms_copy * 1e-3) / 1e9 / HBM_PEAK_GBPS, 1)}
    del rots, part_state, shared
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return res


def summary(res: dict) -> dict:
    """A measured config as the `also` entries carry it: step and kernel figures, roofline."""
    out = {"config": res["config"], "dtype": res["dtype"],
           "us_per_step": round(res["ms_per_step"] * 1e3, 2), "GBps": round(res["value"], 1),
           "pct_peak_hbm": res["pct_peak_hbm"], "tokens_per_s": res["tokens_per_s"],
           "roofline": res["roofline"]}
    for key in ("kv_append", "kv_append_fp8", "copy_blocks"):
        if key in res:
            out[key] = res[key]
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--config", type=int, default=None,
                    help="measure this config alone (default: config 2, the headline, with "
                         "every other config beside it)")
    ap.add_argument("--partition", type=int, default=0,
                    help="a fixed split-KV partition length in keys (0: the library's split of "
                         "each sequence by its own length)")
    ap.add_argument("--max-seq-len", type=int, default=0,
                    help="pad block tables to kelpie's width for this max_seq_len (0: as wide as "
                         "the batch needs)")
    ap.add_argument("--members", type=int, default=2,
                    help="layers in the arena's unit (the row stride spans them all)")
    ap.add_argument("--cases", action="store_true",
                    help="instead of the configs: microseconds per layer for the reference's "
                         "timing buckets (kelpie/scripts/bench_attention.py), with its published "
                         "A100/H100 figures beside them")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": f"--gpus {args.gpus}: this build measures one GPU; the paged-KV "
                                   "path shards by kv head / by sequence with no exchange, and "
                                   "no multi-GPU figure is produced"}))
        return 2

    import torch

    torch.cuda.set_device(0)
    if args.cases:
        print(json.dumps(reference_buckets_line()), flush=True)
        return 0
    cfg = args.config or CONFIG
    res = measure(cfg, args, extras=True)
    line = {
        "metric": METRIC,
        "value": round(res["value"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": res["dtype"],
        "data": f"synthetic (seeded; N(0,1) rounded to bf16, random page tables over a "
                f"{res['pool_pages']}-page pool, {ROTATE} rotating pools)",
        "config": res["config"],
        "pct_peak_hbm": res["pct_peak_hbm"],
        "tokens_per_s": res["tokens_per_s"],
        "tokens_per_s_32_layers": res["tokens_per_s_32_layers"],
        "step_bytes": res["step_bytes"],
        "roofline": res["roofline"],
    }
    for key in ("kv_append", "kv_append_fp8", "copy_blocks"):
        if key in res:
            line[key] = res[key]
    if cfg == CONFIG:
        # The targets this config is judged by, each with the figure it is read from: decode
        # attention is the whole step (split-KV partitions + reduce, the append fused in), the
        # append its bandwidth-sized step. The partition kernel alone is roofline.frac.
        line["gates"] = {
            "decode_attention": {"pct_peak_hbm": res["pct_peak_hbm"], "target": 70.0,
                                 "from": "pct_peak_hbm (the whole step)"},
            "kv_append": {"pct_peak_hbm": res["kv_append"]["pct_peak_hbm"], "target": 60.0,
                          "from": "kv_append.pct_peak_hbm"}}
    if args.config is None:
        line["also"] = {}
        for other in ALSO:
            r = measure(other, args, extras=True)
            line["also"][r["workload"]] = summary(r)
            if other == 10:
                # The same target at the shape it is worded for (batch 64, every context 4k).
                line["gates"]["decode_attention_ctx4k"] = {
                    "pct_peak_hbm": r["pct_peak_hbm"], "target": 70.0,
                    "from": f"also.{r['workload']}.pct_peak_hbm (the whole step)"}
    if not args.no_cpu_baseline:
        log("cpu baseline")
        line["cpu_baseline"] = cpu_baseline(res["batch"], cfg, res["step_bytes"])
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
