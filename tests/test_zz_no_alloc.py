"""kvpath_paged_attention_noalloc: the whole op for callers that cannot allocate (no counterpart in
the reference). Its split-KV partials live in the library's own 64 MiB device scratch.

GPU: two calls in a row through the C ABI -- a decode step, then a smaller verify step -- each
against kvpath_paged_attention with a torch-allocated workspace on an identical copy of the pool:
output and pool bit for bit. CPU: a step whose workspace exceeds the scratch is refused with
EINVAL before any device call.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from kvpath import _lib
from kvpath.paged_attention import _cache, _dtype_code, _opts, _plan, _rows, _stream, _workspace
from workloads import Batch, synthetic

SCRATCH_BYTES = 64 << 20


def _call(step, noalloc: bool, sync: bool = True) -> torch.Tensor:
    """The op on step's pool through the C ABI, with or without a workspace (and, with
    sync=False, without synchronizing: a call that is being captured)."""
    lib = _lib.load()
    q, k, v, kv_member, rr, pos, qsl, lens, table, slots, window, sinks, causal = step.args
    cache = _cache(kv_member, step.kv_scale)
    qr, qq = _rows(q, "q")
    kr, kk = _rows(k, "k")
    vr, vv = _rows(v, "v")
    out = torch.full((q.shape[0], q.shape[1] * q.shape[2]), float("nan"), dtype=q.dtype,
                     device=q.device)
    outr = _lib.Rows(out.data_ptr(), q.shape[0], q.shape[1], q.shape[2], out.stride(0), q.shape[2],
                     _dtype_code(out, "out"))
    plan, keep = _plan(rr, qsl, lens, table, slots, q.shape[0])
    opts, sinks32 = _opts(window, sinks, q.shape[1], causal, 0)
    stream = _stream(q.device)
    if noalloc:
        st = lib.kvpath_paged_attention_noalloc(
            ctypes.byref(qr), ctypes.byref(kr), ctypes.byref(vr), ctypes.byref(cache),
            ctypes.byref(plan), ctypes.byref(opts), ctypes.byref(outr), stream)
        _lib.check("paged_attention_noalloc", st)
    else:
        ws = _workspace(q.device, q.shape[0], lens.shape[0], q.shape[1], kv_member.shape[3],
                        q.shape[2], table.shape[1], kv_member.shape[2], 0)
        st = lib.kvpath_paged_attention(
            ctypes.byref(qr), ctypes.byref(kr), ctypes.byref(vr), ctypes.byref(cache),
            ctypes.byref(plan), ctypes.byref(opts), ctypes.byref(outr), ws.data_ptr(),
            ws.numel(), stream)
        _lib.check("paged_attention", st)
    if sync:
        torch.cuda.synchronize()
    del qq, kk, vv, keep, sinks32
    return out


def _pair(batch: Batch, seed: int):
    kw = dict(seed=seed, pool_pages=4096)
    return synthetic(batch, "cuda", torch.bfloat16, **kw), synthetic(batch, "cuda", torch.bfloat16,
                                                                      **kw)


@pytest.mark.gpu
def test_noalloc_matches_the_workspace_entry_point() -> None:
    """Two calls in a row, the second smaller: a 64-entry decode step (1-4k keys, split-KV with
    the reduce, the append fused), then a 4-entry verify step (16 rows each): output and pool
    equal kvpath_paged_attention's bit for bit."""
    g = torch.Generator().manual_seed(90)
    lens = torch.randint(1024, 4097, (64,), generator=g).tolist()
    decode = Batch(entries=tuple((n - 1, 1) for n in lens), tokens=64, reqs=64, heads=32,
                   kv_heads=8, head_dim=128, block=16, sinks=False)
    verify = Batch(entries=((700, 16), (3000, 16), (40, 16), (1500, 16)), tokens=67, reqs=5,
                   heads=32, kv_heads=8, head_dim=128, block=16, sinks=True)
    for batch, seed in ((decode, 91), (verify, 92)):
        a, b = _pair(batch, seed)
        got = _call(a, noalloc=True)
        want = _call(b, noalloc=False)
        assert torch.equal(got.cpu().view(torch.int16), want.cpu().view(torch.int16))
        assert torch.equal(a.arena.cpu().view(torch.int16), b.arena.cpu().view(torch.int16))
        assert not bool(got[batch.n_rows:].ne(0).any())


# Run in a fresh process, so that its first noalloc call on the device is the captured one.
FIRST_CALL_CAPTURED = r"""
import sys
sys.path[:0] = [{root!r}, {root!r} + "/research-2_amd", {root!r} + "/tests"]
import torch
import test_zz_no_alloc as t
from workloads import Batch
batch = Batch(entries=((700, 1), (3000, 1), (40, 1), (1500, 1), (2047, 1)), tokens=6, reqs=6,
              heads=32, kv_heads=8, head_dim=128, block=16, sinks=False)
a, b = t._pair(batch, 93)
arena0 = a.arena.clone()
stream = torch.cuda.Stream()
stream.wait_stream(torch.cuda.current_stream())
graph = torch.cuda.CUDAGraph()
with torch.cuda.stream(stream), torch.cuda.graph(graph, stream=stream):
    out = t._call(a, noalloc=True, sync=False)
torch.cuda.current_stream().wait_stream(stream)
want = t._call(b, noalloc=False)
for replay in range(3):
    a.arena.copy_(arena0)
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out.cpu().view(torch.int16), want.cpu().view(torch.int16)), replay
    assert torch.equal(a.arena.cpu().view(torch.int16), b.arena.cpu().view(torch.int16)), replay
    eager = t._call(b, noalloc=True)  # eager work between the replays, through the same scratch
    assert torch.equal(eager.cpu().view(torch.int16), want.cpu().view(torch.int16)), replay
print("first call captured: ok", flush=True)
"""


@pytest.mark.gpu
def test_noalloc_first_call_under_capture() -> None:
    """In a fresh process, the first kvpath_paged_attention_noalloc call on the device is made
    inside torch.cuda.graph capture (global mode), so the scratch's address is looked up under
    capture: the capture stays valid, and each of three replays (eager calls in between) gives
    the workspace entry point's output and pool, bit for bit."""
    import subprocess
    import sys
    from pathlib import Path

    root = str(Path(__file__).resolve().parents[1])
    proc = subprocess.run([sys.executable, "-c", FIRST_CALL_CAPTURED.format(root=root)],
                          capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stdout[-2000:] + proc.stderr[-4000:]
    assert "first call captured: ok" in proc.stdout


def test_noalloc_refuses_a_step_beyond_its_scratch() -> None:
    """A step whose split-KV workspace exceeds the 64 MiB scratch is refused with EINVAL and a
    message naming the limit, before any device call (none is made here)."""
    lib = _lib.load()
    T, R, H, hkv, D, width, block = 8192, 1, 32, 8, 128, 2048, 16
    need = lib.kvpath_workspace_bytes(T, R, H, hkv, D, width, block, 0)
    assert need > SCRATCH_BYTES
    q = _lib.Rows(0x1000, T, H, D, H * D, D, _lib.BF16)
    kv = _lib.Rows(0x2000, T, hkv, D, hkv * D, D, _lib.BF16)
    out = _lib.Rows(0x3000, T, H, D, H * D, D, _lib.BF16)
    cache = _lib.Cache(0x4000, 4096, block, hkv, D, block * 2 * hkv * D, hkv * D, 2 * hkv * D, D,
                       _lib.BF16, None)
    plan = _lib.Plan(0x10, 0x20, 0x30, 0x40, 0x50, T, R, width, width)
    opts = _lib.AttnOpts(0, None, 1, 0)
    st = lib.kvpath_paged_attention_noalloc(ctypes.byref(q), ctypes.byref(kv), ctypes.byref(kv),
                                            ctypes.byref(cache), ctypes.byref(plan),
                                            ctypes.byref(opts), ctypes.byref(out), None)
    assert st == _lib.EINVAL
    message = lib.kvpath_last_error()
    assert b"67108864" in message and b"kvpath_paged_attention" in message
