"""`kvpath::paged_attention` -- Kelpie's paged-KV op on MI355X HIP kernels.

The host-side mirror of kelpie's op (kelpie/kelpie-models/kelpie_models/kernels/ops/
paged_attention.py): the same names, argument meanings, layout, plan contract and error
behaviour, with every tensor operation replaced by a call through the C ABI of libkvpath.so
(include/kvpath.h). Nothing here computes on the CPU and nothing falls back: a tensor that is not
on a ROCm device, a missing library, or a case no kernel serves raises.

KV LAYOUT (ops/paged_attention.py:3-8): a layer's cache member is `[pages, 2, block, Hkv, D]`,
K = member[:, 0], V = member[:, 1]; any strides (the engine's arena views interleave K/V per row
and span all layers per row, sdk/kv.py:163-224) as long as D is innermost. fp8 adds a scale
tensor f32[pages, 2, Hkv] (`new_kv_scale`).

PLAN (ops/paged_attention.py:10-13, 87-102): int32 `row_request[T]`, `positions[T]`,
`query_start_loc[R+1]`, `seq_lens[R]`, `block_table[R, P]`, `slot_mapping[T]`. The kernels derive
a row's position as seq_lens[r] - rows_r + i (as the vLLM adapter does, kernels/adapters/
paged_attention_vllm.py:59-64) and check `positions` against it on every call, as kelpie's op
asserts it on every call (ops/paged_attention.py:128, 143-157): a row that breaks the plan is
written as NaN and sets this device's plan-status word (`plan_status`, `check_plan_status`);
nothing synchronizes and nothing traps, so the check sits in captured steps too.

The two ops, torch.ops.kvpath.paged_attention and paged_attention_fp8, are registered in C++
(csrc/kvpath_torch.cpp, built into libkvpath_torch.so beside libkvpath.so): the dispatcher calls
the C ABI with no Python frame between the caller and the launch; so are write_kv and
write_kv_fp8, which `write_kv` calls. Their fake (meta) rules are registered here. The other
entry points (attend, kv_gather, copy_blocks) bind the C ABI through ctypes (_lib).
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

from kvpath import _lib

KV_MEMBERS = 2
TORCH_OPS = Path(__file__).resolve().parent / "libkvpath_torch.so"


def _load_ops() -> None:
    """Register torch.ops.kvpath (libkvpath_torch.so, linked to libkvpath.so); raises, naming the
    build command, when either library is missing."""
    _lib.load()
    if not TORCH_OPS.exists():
        raise RuntimeError(f"{TORCH_OPS.name} not found at {TORCH_OPS}: build it first "
                           f"(python -c 'import __graft_entry__ as g; g.build()' at the repo root)")
    torch.ops.load_library(str(TORCH_OPS))


_load_ops()


def set_slot_check(on: bool) -> bool:
    """Turn the plan check's slot comparison on or off for later op calls (every thread);
    returns the old setting. It compares each fused-append row's slot_mapping with its position's
    slot in the block table, one more dependent load per row in the output writers, so it is off
    unless KVPATH_CHECK_SLOTS=1 or this turns it on; the position check always runs."""
    return bool(torch.ops.kvpath.set_check_slots(bool(on)))


set_slot_check(os.environ.get("KVPATH_CHECK_SLOTS", "0") == "1")

_DTYPES = {
    torch.float32: _lib.F32,
    torch.float16: _lib.F16,
    torch.bfloat16: _lib.BF16,
    torch.float8_e4m3fn: _lib.FP8_E4M3,
}


def _dtype_code(t: torch.Tensor, what: str) -> int:
    code = _DTYPES.get(t.dtype)
    if code is None:
        raise NotImplementedError(f"kvpath: {what} dtype {t.dtype} (serves f32, f16, bf16, "
                                  f"float8_e4m3fn caches)")
    return code


def _on_device(*tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    for t in tensors:
        if t.device.type != "cuda" or t.device != dev:
            raise RuntimeError(
                f"kvpath: every tensor must be on one ROCm device, got {t.device} (and {dev}); "
                f"there is no CPU path")
    return dev


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def kv_views(kv_member: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """The member `[pages, 2, block, Hkv, D]` as K and V, each `[pages * block, Hkv, D]`
    (ops/paged_attention.py:27-41). Fails when the reshape would copy rather than view."""
    pages, two, block, heads, dim = kv_member.shape
    assert two == KV_MEMBERS, kv_member.shape
    k, v = (kv_member[:, i].reshape(pages * block, heads, dim) for i in range(KV_MEMBERS))
    assert k.untyped_storage().data_ptr() == kv_member.untyped_storage().data_ptr(), (
        "kv member layout does not flatten to a view", kv_member.shape, kv_member.stride())
    return k, v


def no_sinks(like: torch.Tensor) -> torch.Tensor:
    """The `sinks` argument for a model without attention sinks (ops/paged_attention.py:243-245)."""
    return torch.empty(0, dtype=torch.float32, device=like.device)


def new_kv_scale(kv_member: torch.Tensor) -> torch.Tensor:
    """The per-(page, K/V, kv-head) dequant scales of an fp8 member: f32[pages, 2, Hkv], zeros."""
    pages, _, _, heads, _ = kv_member.shape
    return torch.zeros(pages, KV_MEMBERS, heads, dtype=torch.float32, device=kv_member.device)


# ---- ctypes views of tensors --------------------------------------------------------------------


def _cache(kv_member: torch.Tensor, kv_scale: torch.Tensor | None) -> _lib.Cache:
    if kv_member.dim() != 5 or kv_member.shape[1] != KV_MEMBERS:
        raise ValueError(f"kv_member must be [pages, 2, block, Hkv, D], got {tuple(kv_member.shape)}")
    if kv_member.stride(-1) != 1:
        raise NotImplementedError(f"kvpath: kv_member's D stride is {kv_member.stride(-1)}, "
                                  f"kernels need D innermost")
    code = _dtype_code(kv_member, "kv_member")
    pages, _, block, heads, dim = kv_member.shape
    s_page, s_kv, s_row, s_head, _ = kv_member.stride()
    scale = None
    if code == _lib.FP8_E4M3:
        if kv_scale is None:
            raise ValueError("kvpath: an fp8 kv_member needs kv_scale (new_kv_scale)")
        if (kv_scale.dtype != torch.float32 or tuple(kv_scale.shape) != (pages, KV_MEMBERS, heads)
                or not kv_scale.is_contiguous()):
            raise ValueError(f"kvpath: kv_scale must be contiguous f32[{pages}, 2, {heads}], got "
                             f"{kv_scale.dtype} {tuple(kv_scale.shape)}")
        scale = kv_scale.data_ptr()
    return _lib.Cache(kv_member.data_ptr(), pages, block, heads, dim, s_page, s_kv, s_row, s_head,
                      code, scale)


def _rows(x: torch.Tensor, what: str) -> tuple[_lib.Rows, torch.Tensor]:
    """A [T, heads, D] tensor as kvpath_rows; a tensor whose D is not innermost is copied."""
    if x.dim() != 3:
        raise ValueError(f"kvpath: {what} must be [T, heads, D], got {tuple(x.shape)}")
    if x.stride(-1) != 1:
        x = x.contiguous()
    return _lib.Rows(x.data_ptr(), x.shape[0], x.shape[1], x.shape[2], x.stride(0), x.stride(1),
                     _dtype_code(x, what)), x


def _plan(row_request, query_start_loc, seq_lens, block_table, slot_mapping, n_tokens: int,
          positions=None) -> tuple[_lib.Plan, tuple[torch.Tensor, ...]]:
    keep = []

    def i32(t: torch.Tensor | None, what: str) -> torch.Tensor | None:
        if t is None:
            return None
        if t.dtype != torch.int32:
            raise ValueError(f"kvpath: {what} must be int32 (sdk/device.py casts the plan to i32), "
                             f"got {t.dtype}")
        if what == "block_table":
            if t.dim() != 2:
                raise ValueError(f"kvpath: block_table must be [R, P], got {tuple(t.shape)}")
            if t.stride(1) != 1 or t.stride(0) < t.shape[1]:
                t = t.contiguous()
        elif not t.is_contiguous():
            t = t.contiguous()
        keep.append(t)
        return t

    def ptr(t: torch.Tensor | None) -> int | None:
        return None if t is None else t.data_ptr()

    # The plan's lengths (ops/paged_attention.py:90-101): the kernels read these tensors through
    # bare pointers, so one of another length is refused instead of being read past its end.
    for t, what in ((row_request, "row_request"), (positions, "positions"),
                    (slot_mapping, "slot_mapping")):
        if t is not None and (t.dim() != 1 or t.shape[0] != n_tokens):
            raise ValueError(f"kvpath: {what} must be i32[T = {n_tokens}], got {tuple(t.shape)}")
    if seq_lens is not None:
        if seq_lens.dim() != 1:
            raise ValueError(f"kvpath: seq_lens must be i32[R], got {tuple(seq_lens.shape)}")
        n = seq_lens.shape[0]
        if query_start_loc is not None and (query_start_loc.dim() != 1 or
                                            query_start_loc.shape[0] != n + 1):
            raise ValueError(f"kvpath: query_start_loc must be i32[R + 1 = {n + 1}], got "
                             f"{tuple(query_start_loc.shape)}")
        if block_table is not None and (block_table.dim() != 2 or block_table.shape[0] != n):
            raise ValueError(f"kvpath: block_table must be i32[R = {n}, P], got "
                             f"{tuple(block_table.shape)}")
    table = i32(block_table, "block_table")
    n_reqs = seq_lens.shape[0] if seq_lens is not None else 0
    width = table.shape[1] if table is not None else 0
    plan = _lib.Plan(
        ptr(i32(row_request, "row_request")), ptr(i32(query_start_loc, "query_start_loc")),
        ptr(i32(seq_lens, "seq_lens")), ptr(table), ptr(i32(slot_mapping, "slot_mapping")),
        n_tokens, n_reqs, width, max(table.stride(0), width) if table is not None else width,
        ptr(i32(positions, "positions")))
    return plan, tuple(keep)


def _workspace(device: torch.device, n_tokens: int, n_reqs: int, n_heads: int, kv_heads: int,
               head_dim: int, width: int, block: int, partition: int) -> torch.Tensor:
    size = _lib.load().kvpath_workspace_bytes(n_tokens, n_reqs, n_heads, kv_heads, head_dim, width,
                                              block, partition)
    if size < 0:
        raise ValueError("kvpath: bad workspace shape")
    ws = torch.empty(size + 256, dtype=torch.uint8, device=device)
    off = (-ws.data_ptr()) % 256
    return ws[off: off + size] if size > 0 else ws[:1]


def _opts(window: int, sinks: torch.Tensor, n_heads: int, causal: bool, partition: int,
          status: int | None = None) -> tuple[_lib.AttnOpts, torch.Tensor]:
    sink_ptr = None
    if sinks.numel() > 0:
        if sinks.shape != (n_heads,):
            raise ValueError(f"kvpath: sinks must be f32[{n_heads}], got {tuple(sinks.shape)}")
        sinks = sinks.to(torch.float32).contiguous()
        sink_ptr = sinks.data_ptr()
    return _lib.AttnOpts(int(window), sink_ptr, int(bool(causal)), int(partition), status), sinks


def _device_index(device: torch.device | int | None) -> int:
    if isinstance(device, int):
        return device
    if device is None or device.index is None:
        return torch.cuda.current_device()
    return device.index


def _status_word(device: torch.device | int | None) -> torch.Tensor:
    """This device's plan-status word: an int32 the kernels' plan check ORs 1 into, created
    (zeroed) by the op's first call on the device outside graph capture, or here."""
    return torch.ops.kvpath.plan_status_word(_device_index(device))


def plan_status(device: torch.device | int | None = None) -> int:
    """The bits the kernels' plan check has set on this device since the last clear (0: every
    checked row was its entry's newest position at its table slot). Synchronizes the device."""
    word = _status_word(device)
    torch.cuda.synchronize(word.device)
    return int(word.item())


def clear_plan_status(device: torch.device | int | None = None) -> None:
    """Zero this device's plan-status word (synchronously)."""
    word = _status_word(device)
    torch.cuda.synchronize(word.device)
    word.zero_()
    torch.cuda.synchronize(word.device)


def check_plan_status(device: torch.device | int | None = None) -> None:
    """Raise if a call on this device broke the plan (kelpie's op fails its stream on the same
    condition, ops/paged_attention.py:143-157; here the caller picks where it surfaces)."""
    bits = plan_status(device)
    if bits:
        raise RuntimeError(f"kvpath: a paged_attention call broke the plan (status {bits:#x}): "
                           f"some row is not its entry's newest position, or its slot_mapping "
                           f"is not that position's table slot; its output rows are NaN")


def assert_newest_positions(row_request: torch.Tensor, positions: torch.Tensor,
                            query_start_loc: torch.Tensor, seq_lens: torch.Tensor) -> None:
    """kelpie's plan invariant as kelpie asserts it (ops/paged_attention.py:143-157): every live
    row t of entry r lies in [qsl[r], qsl[r+1]) and positions[t] == seq_lens[r] - rows_r +
    (t - qsl[r]). Checked with torch._assert_async on the tensors' device: no host sync, so it
    can sit in a captured step; a violation fails the stream (or raises at once on CPU tensors).
    The op itself does not call it: its kernels check the same invariant on every call and
    answer a violation with NaN rows and the plan-status word (plan_status), which never traps;
    this is for a caller that wants kelpie's failing stream instead."""
    live = row_request >= 0
    entry = row_request.clamp(min=0).long()
    t = torch.arange(row_request.shape[0], device=row_request.device)
    start = query_start_loc.long()[entry]
    stop = query_start_loc.long()[entry + 1]
    want = seq_lens.long()[entry] - (stop - start) + (t - start)
    ok = (t >= start) & (t < stop) & (positions.long() == want)
    torch._assert_async(torch.all(ok | ~live), "plan rows are not their entry's newest positions")


def split_plan(n_tokens: int, n_reqs: int, n_heads: int, kv_heads: int, width: int, block: int,
               partition: int = 0) -> tuple[int, int, bool]:
    """How the library splits a step of this shape into split-KV partitions (kvpath_split_plan):
    (partition_tokens, slots, per_entry). With `partition` 0 each entry's keys are cut on the
    device, from its own seq_len, into min(slots, ceil(span / partition_tokens)) equal partitions
    rounded up to 32 keys; with `partition` > 0 every partition has that length."""
    out = _lib.Split()
    _lib.check("split_plan", _lib.load().kvpath_split_plan(n_tokens, n_reqs, n_heads, kv_heads,
                                                           width, block, int(partition),
                                                           ctypes.byref(out)))
    return out.partition_tokens, out.slots, bool(out.per_entry)


def workspace_bytes(n_tokens: int, n_reqs: int, n_heads: int, kv_heads: int, head_dim: int,
                    width: int, block: int, partition: int = 0) -> int:
    """Bytes of split-KV scratch one attention call of this shape needs (kvpath_workspace_bytes)
    at `partition` (0: the library's split)."""
    return _lib.load().kvpath_workspace_bytes(n_tokens, n_reqs, n_heads, kv_heads, head_dim, width,
                                              block, partition)


def workspace_bytes_max(max_tokens: int, max_reqs: int, n_heads: int, kv_heads: int,
                        head_dim: int, width: int, block: int, partition: int = 0) -> int:
    """Bytes of split-KV scratch that serve every step of at most `max_tokens` rows and
    `max_reqs` entries of this shape (kvpath_workspace_bytes_max): one allocation for a largest
    bucket covers the smaller ones, which workspace_bytes of the largest shape alone does not."""
    return _lib.load().kvpath_workspace_bytes_max(max_tokens, max_reqs, n_heads, kv_heads,
                                                  head_dim, width, block, partition)


# ---- entry points -------------------------------------------------------------------------------


def write_kv(kv_member: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
             slot_mapping: torch.Tensor, kv_scale: torch.Tensor | None = None) -> None:
    """Scatter k, v [T, Hkv, D] into the member at flat slots (ops/paged_attention.py:44-54),
    converting to the cache dtype; with an fp8 member, quantize on append and update kv_scale.
    (torch.ops.kvpath.write_kv / write_kv_fp8, registered in C++ over kvpath_kv_append.)"""
    if kv_member.dtype == torch.float8_e4m3fn:
        if kv_scale is None:
            raise ValueError("kvpath: an fp8 kv_member needs kv_scale (new_kv_scale)")
        torch.ops.kvpath.write_kv_fp8(kv_member, k, v, slot_mapping, kv_scale)
    else:
        torch.ops.kvpath.write_kv(kv_member, k, v, slot_mapping)


@torch.library.register_fake("kvpath::write_kv")
def _fake_write_kv(kv_member, k, v, slot_mapping):
    del kv_member, k, v, slot_mapping


@torch.library.register_fake("kvpath::write_kv_fp8")
def _fake_write_kv_fp8(kv_member, k, v, slot_mapping, kv_scale):
    del kv_member, k, v, slot_mapping, kv_scale


def attend(q: torch.Tensor, kv_member: torch.Tensor, row_request: torch.Tensor,
           query_start_loc: torch.Tensor, seq_lens: torch.Tensor, block_table: torch.Tensor,
           window: int, sinks: torch.Tensor, causal: bool = True,
           kv_scale: torch.Tensor | None = None, partition: int = 0,
           out: torch.Tensor | None = None) -> torch.Tensor:
    """Attention only, over pages already written (ops/paged_attention.py:160-240 for the whole
    plan): -> [T, H * D] in q.dtype, pad rows zero."""
    dev = _on_device(q, kv_member, row_request, query_start_loc, seq_lens, block_table)
    lib = _lib.load()
    n_tokens, n_heads, head_dim = q.shape
    cache = _cache(kv_member, kv_scale)
    qr, qq = _rows(q, "q")
    if out is None:
        out = torch.empty(n_tokens, n_heads * head_dim, dtype=q.dtype, device=dev)
    outr = _lib.Rows(out.data_ptr(), n_tokens, n_heads, head_dim, out.stride(0), head_dim,
                     _dtype_code(out, "out"))
    plan, keep = _plan(row_request, query_start_loc, seq_lens, block_table, None, n_tokens)
    opts, sinks = _opts(window, sinks, n_heads, causal, max(0, int(partition)))
    ws = _workspace(dev, n_tokens, seq_lens.shape[0], n_heads, kv_member.shape[3], head_dim,
                    block_table.shape[1], kv_member.shape[2], max(0, int(partition)))
    with torch.cuda.device(dev):
        _lib.check("attend", lib.kvpath_attend(ctypes.byref(qr), ctypes.byref(cache),
                                               ctypes.byref(plan), ctypes.byref(opts),
                                               ctypes.byref(outr), ws.data_ptr(), ws.numel(),
                                               _stream(dev)))
    del qq, keep
    return out


# kelpie::paged_attention's contract (ops/paged_attention.py:67-109) on HIP, registered in C++:
# append k/v at slot_mapping into `kv_member` (in place), then paged causal GQA attention ->
# [T, H * D] in q.dtype, pad rows exactly zero. Same 13 arguments, same order and meaning; the
# optional trailing `partition` (split-KV partition length in keys, 0 = the library's split of
# each entry by its own length) is this build's tuning knob and changes no result beyond fp32
# rounding. paged_attention_fp8 takes the 13 arguments plus an fp8 member's scales
# f32[pages, 2, Hkv] (`new_kv_scale`): k/v are quantized on append, dequantized in-kernel.
# Backward raises NotImplementedError: the op is inference-only, as kelpie's is
# (ops/paged_attention.py:380-385).
paged_attention = torch.ops.kvpath.paged_attention
paged_attention_fp8 = torch.ops.kvpath.paged_attention_fp8


@torch.library.register_fake("kvpath::paged_attention")
def _fake(q, k, v, kv_member, row_request, positions, query_start_loc, seq_lens, block_table,
          slot_mapping, window, sinks, causal=True, partition=0):
    """The shape rule (ops/paged_attention.py:248-267): [T, H * D] in q's dtype."""
    del k, v, kv_member, row_request, positions, query_start_loc, seq_lens, block_table
    del slot_mapping, window, sinks, causal, partition
    return torch.empty(q.shape[0], q.shape[1] * q.shape[2], dtype=q.dtype, device=q.device)


@torch.library.register_fake("kvpath::paged_attention_fp8")
def _fake_fp8(q, k, v, kv_member, row_request, positions, query_start_loc, seq_lens, block_table,
              slot_mapping, window, sinks, causal, kv_scale, partition=0):
    del k, v, kv_member, row_request, positions, query_start_loc, seq_lens, block_table
    del slot_mapping, window, sinks, causal, kv_scale, partition
    return torch.empty(q.shape[0], q.shape[1] * q.shape[2], dtype=q.dtype, device=q.device)


def kv_gather(kv_member: torch.Tensor, block_table: torch.Tensor, width: int | None = None
              ) -> tuple[torch.Tensor, torch.Tensor]:
    """The gather inside _attend (ops/paged_attention.py:172-177): K and V of every entry's first
    `width` pages as dense [R, width * block, Hkv, D] in the cache dtype, bit-exact."""
    dev = _on_device(kv_member, block_table)
    lib = _lib.load()
    pages, _, block, heads, dim = kv_member.shape
    width = block_table.shape[1] if width is None else int(width)
    cache = _cache(kv_member, torch.zeros(pages, KV_MEMBERS, heads, device=dev)
                   if kv_member.dtype == torch.float8_e4m3fn else None)
    plan, keep = _plan(None, None, None, block_table, None, 0)
    plan.num_reqs = block_table.shape[0]
    out_k = torch.empty(block_table.shape[0], width * block, heads, dim, dtype=kv_member.dtype,
                        device=dev)
    out_v = torch.empty_like(out_k)
    with torch.cuda.device(dev):
        _lib.check("kv_gather", lib.kvpath_kv_gather(ctypes.byref(cache), ctypes.byref(plan), width,
                                                     out_k.data_ptr(), out_v.data_ptr(),
                                                     _stream(dev)))
    del keep
    return out_k, out_v


def copy_blocks(kv_member: torch.Tensor, src: torch.Tensor, dst: torch.Tensor,
                kv_scale: torch.Tensor | None = None) -> None:
    """Page dst[i] <- page src[i] (every row, K and V, and an fp8 member's scales). dst ids must
    be distinct and disjoint from the src ids. src, dst: int32 device tensors [N]."""
    dev = _on_device(kv_member, src, dst)
    lib = _lib.load()
    if src.shape != dst.shape or src.dim() != 1:
        raise ValueError(f"kvpath: src {tuple(src.shape)} and dst {tuple(dst.shape)} must be [N]")
    if src.dtype != torch.int32 or dst.dtype != torch.int32:
        raise ValueError("kvpath: copy_blocks page ids must be int32")
    src, dst = src.contiguous(), dst.contiguous()
    cache = _cache(kv_member, kv_scale)
    with torch.cuda.device(dev):
        _lib.check("copy_blocks", lib.kvpath_copy_blocks(ctypes.byref(cache), src.data_ptr(),
                                                         dst.data_ptr(), src.shape[0],
                                                         _stream(dev)))
