"""The C ABI (include/kvpath.h) without a GPU: libkvpath.so loads, exports every function the
header declares with the binding's signature, and its validation layer refuses bad arguments
with the documented status and message before touching a device.
"""

from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest
import torch

import kvpath
from kvpath import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "kvpath.h"


@pytest.fixture(scope="module")
def lib() -> ctypes.CDLL:
    if not _lib.LIBRARY.exists():
        from kvpath import build

        build.build()
    return _lib.load()


def header_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(kvpath_[a-z_0-9]+)\s*\(", text,
                      flags=re.M)


def test_header_and_binding_agree() -> None:
    assert header_functions() == list(_lib.EXPORTS)


def test_library_exports_every_symbol(lib) -> None:
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIBRARY)], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    for name in header_functions():
        assert name in exported, name
        assert getattr(lib, name) is not None
    assert lib.kvpath_abi_version() == _lib.ABI_VERSION


def test_workspace_bytes(lib) -> None:
    # C2 at a fixed 512-key partition: T 64, H 32, D 128, table width 256 pages of 16 -> 8 slots
    n = lib.kvpath_workspace_bytes(64, 64, 32, 8, 128, 256, 16, 512)
    parts = 8
    o = 64 * 32 * parts * 128 * 4
    assert n == (o + 255) // 256 * 256 + 64 * 32 * parts * 2 * 4
    assert lib.kvpath_workspace_bytes(64, 64, 32, 8, 128, 256, 16, 100) == -1  # not x 32
    assert lib.kvpath_workspace_bytes(64, 64, 30, 8, 128, 256, 16, 0) == -1  # 30 q / 8 kv heads
    assert kvpath.workspace_bytes(4, 4, 64, 8, 128, 8192, 16) == lib.kvpath_workspace_bytes(
        4, 4, 64, 8, 128, 8192, 16, 0)
    # The library's split: nine slots at config 2 however wide kelpie makes the table.
    nine = 64 * 32 * 9
    want = (nine * 128 * 4 + 255) // 256 * 256 + nine * 8
    for width in (258, 512, 8192):
        assert lib.kvpath_workspace_bytes(64, 64, 32, 8, 128, width, 16, 0) == want


def _cache(**kw) -> _lib.Cache:
    c = dict(base=0x1000, num_pages=8, block_size=16, num_kv_heads=2, head_dim=64,
             stride_page=16 * 2 * 2 * 64, stride_kv=2 * 64, stride_row=2 * 2 * 64,
             stride_head=64, dtype=_lib.BF16, scale=None)
    c.update(kw)
    return _lib.Cache(**c)


@pytest.mark.parametrize("shape,want", [
    ((64, 64, 32, 8, 258, 16, 0), (512, 9, 1)),      # decode (config 2)
    ((64, 64, 32, 8, 512, 16, 0), (512, 9, 1)),      # ... at kelpie's width for max_seq_len 8k
    ((64, 64, 32, 8, 8192, 16, 0), (512, 9, 1)),     # ... and for 128k: the same grid
    ((256, 16, 32, 8, 514, 16, 0), (896, 9, 1)),     # verify, 16 rows per entry (config 3)
    ((256, 16, 32, 8, 8192, 16, 0), (896, 9, 1)),    # ... at kelpie's 128k width
    ((1024, 64, 32, 8, 514, 16, 0), (896, 9, 1)),    # verify over 64 entries
    ((4, 4, 64, 8, 8194, 16, 0), (512, 65, 1)),      # 128k decode (config 5): 2048+ workgroups
    ((128, 128, 32, 8, 513, 16, 0), (512, 9, 1)),    # fp8 decode over 2-8k keys (config 4)
    ((2048, 4, 32, 8, 160, 16, 0), (512, 1, 1)),     # prefill, 512-row chunks after 2k keys
    ((8192, 1, 32, 8, 2048, 16, 0), (512, 3, 1)),    # one long prefill chunk: 1024 workgroups
    ((64, 64, 32, 8, 3, 16, 0), (512, 1, 1)),        # a table of 48 keys: one slot
    ((64, 64, 32, 8, 34, 16, 0), (512, 1, 1)),       # decode over 544 keys: one partition each
    ((8, 8, 64, 8, 45, 16, 0), (512, 1, 1)),         # gpt-oss decode over 720 keys: the same
    ((8, 8, 32, 8, 64, 16, 0), (512, 2, 1)),         # decode over 1024 keys: split again
    ((0, 0, 32, 8, 1, 16, 0), (512, 1, 1)),          # empty step
    ((4, 4, 64, 8, 8192, 16, 512), (512, 256, 0)),   # a fixed 512: 256 partitions of 128k
    ((64, 64, 32, 8, 258, 16, 480), (480, 9, 0)),    # a fixed 480 over 4128 keys
])
def test_split_choice(lib, shape, want) -> None:
    """The library's split-KV plan. With partition 0, each entry is cut on the device by its own
    length: a floor of 512 keys (896 for verify-shaped steps), at most `slots` partitions per
    entry, where the slots give the grid 2048+ workgroups (decode) or 1024+ (verify), at least
    nine, an odd count, and never more than the table could fill at the floor; a decode step
    over at most 768 keys takes one slot (one partition per entry, no reduce); prefill-sized
    steps fill the grid with rows and take slots only up to 1024 workgroups. A fixed partition
    length gives ceil(keys / length) slots."""
    T, R, H, hkv, width, block, part = shape
    out = _lib.Split()
    assert lib.kvpath_split_plan(T, R, H, hkv, width, block, part, ctypes.byref(out)) == _lib.OK
    assert (out.partition_tokens, out.slots, out.per_entry) == want
    assert kvpath.split_plan(T, R, H, hkv, width, block, part) == (want[0], want[1], bool(want[2]))


def test_validation_refuses_before_any_launch(lib) -> None:
    """Null / inconsistent arguments return EINVAL with a message; no device is touched (there
    is none here), so the checks run entirely on the host."""
    rows = _lib.Rows(0x2000, 4, 2, 64, 128, 64, _lib.BF16)
    plan = _lib.Plan(None, None, None, None, None, 4, 1, 1, 1)
    null = _lib.Cache()
    assert lib.kvpath_kv_append(ctypes.byref(null), ctypes.byref(rows), ctypes.byref(rows),
                                ctypes.byref(plan), None) == _lib.EINVAL
    assert b"null cache" in lib.kvpath_last_error()

    cache = _cache()
    st = lib.kvpath_kv_append(ctypes.byref(cache), ctypes.byref(rows), ctypes.byref(rows),
                              ctypes.byref(plan), None)
    assert st == _lib.EINVAL and b"slot_mapping" in lib.kvpath_last_error()

    bad_rows = _lib.Rows(0x2000, 4, 3, 64, 192, 64, _lib.BF16)  # 3 heads, cache has 2
    st = lib.kvpath_kv_append(ctypes.byref(cache), ctypes.byref(bad_rows), ctypes.byref(rows),
                              ctypes.byref(plan), None)
    assert st == _lib.EINVAL and b"want [4, 2, 64]" in lib.kvpath_last_error()

    fp8 = _cache(dtype=_lib.FP8_E4M3)
    st = lib.kvpath_copy_blocks(ctypes.byref(fp8), None, None, 0, None)
    assert st == _lib.EINVAL and b"scale" in lib.kvpath_last_error()

    q = _lib.Rows(0x2000, 4, 3, 64, 192, 64, _lib.BF16)  # 3 q heads over 2 kv heads
    out = _lib.Rows(0x3000, 4, 3, 64, 192, 64, _lib.BF16)
    opts = _lib.AttnOpts(0, None, 1, 512)
    st = lib.kvpath_attend(ctypes.byref(q), ctypes.byref(cache), ctypes.byref(plan),
                           ctypes.byref(opts), ctypes.byref(out), None, 0, None)
    assert st == _lib.EINVAL and b"not a multiple" in lib.kvpath_last_error()

    q = _lib.Rows(0x2000, 4, 4, 64, 256, 64, _lib.BF16)
    out = _lib.Rows(0x3000, 4, 4, 64, 256, 64, _lib.BF16)
    full = _lib.Plan(0x10, 0x20, 0x30, 0x40, 0x50, 4, 2, 3, 3)
    st = lib.kvpath_attend(ctypes.byref(q), ctypes.byref(cache), ctypes.byref(full),
                           ctypes.byref(opts), ctypes.byref(out), None, 0, None)
    assert st == _lib.EINVAL and b"workspace" in lib.kvpath_last_error()

    odd = _lib.AttnOpts(0, None, 1, 100)
    st = lib.kvpath_attend(ctypes.byref(q), ctypes.byref(cache), ctypes.byref(full),
                           ctypes.byref(odd), ctypes.byref(out), None, 0, None)
    assert st == _lib.EINVAL and b"multiple of 32" in lib.kvpath_last_error()


def test_oversized_shapes_are_refused(lib) -> None:
    """Sizes whose products would overflow int64, or that the kernels' int32 fields cannot
    hold, are refused on the host before any product is formed: workspace_bytes returns -1, the
    entry points EINVAL."""
    ws = lib.kvpath_workspace_bytes  # (T, R, H, Hkv, D, width, block, partition)
    assert ws(1 << 31, 1, 32, 8, 128, 256, 16, 512) == -1
    assert ws(64, 1 << 16, 32, 8, 128, 256, 16, 512) == -1
    assert ws(64, 1, 1 << 20, 1, 128, 256, 16, 512) == -1
    assert ws(64, 1, 32, 8, 1 << 20, 256, 16, 512) == -1
    assert ws(64, 1, 32, 8, 128, 1 << 40, 16, 512) == -1
    assert ws(64, 1, 32, 8, 128, 1 << 27, 1 << 8, 512) == -1
    assert ws((1 << 31) - 1, 1, 1 << 16, 1 << 16, 1 << 16, 4096, 16, 32) == -1
    rows_parts = (1 << 20) * 64 * 8  # 256 x 16 keys in 512-key partitions
    assert ws(1 << 20, 1, 64, 8, 128, 256, 16, 512) == rows_parts * 128 * 4 + rows_parts * 8

    rows = _lib.Rows(0x2000, 4, 2, 64, 128, 64, _lib.BF16)
    plan = _lib.Plan(0x10, 0x20, 0x30, 0x40, 0x50, 4, 2, 3, 3)
    wide = _cache(head_dim=1 << 20)
    st = lib.kvpath_kv_append(ctypes.byref(wide), ctypes.byref(rows), ctypes.byref(rows),
                              ctypes.byref(plan), None)
    assert st == _lib.EINVAL and b"exceed" in lib.kvpath_last_error()
    huge = _cache(num_pages=1 << 40, block_size=1 << 30)
    st = lib.kvpath_kv_append(ctypes.byref(huge), ctypes.byref(rows), ctypes.byref(rows),
                              ctypes.byref(plan), None)
    assert st == _lib.EINVAL and b"int32 slot mapping" in lib.kvpath_last_error()

    cache = _cache()
    opts = _lib.AttnOpts(0, None, 1, 512)
    many = _lib.Rows(0x2000, 4, 1 << 20, 64, (1 << 20) * 64, 64, _lib.BF16)
    st = lib.kvpath_attend(ctypes.byref(many), ctypes.byref(cache), ctypes.byref(plan),
                           ctypes.byref(opts), ctypes.byref(many), None, 0, None)
    assert st == _lib.EINVAL and b"q heads exceed" in lib.kvpath_last_error()
    q = _lib.Rows(0x2000, 4, 4, 64, 256, 64, _lib.BF16)
    long_table = _lib.Plan(0x10, 0x20, 0x30, 0x40, 0x50, 4, 2, 1 << 40, 1 << 40)
    st = lib.kvpath_attend(ctypes.byref(q), ctypes.byref(cache), ctypes.byref(long_table),
                           ctypes.byref(opts), ctypes.byref(q), None, 0, None)
    assert st == _lib.EINVAL and b"too many keys" in lib.kvpath_last_error()
    back = _lib.AttnOpts(-5, None, 1, 512)
    st = lib.kvpath_attend(ctypes.byref(q), ctypes.byref(cache), ctypes.byref(plan),
                           ctypes.byref(back), ctypes.byref(q), None, 0, None)
    assert st == _lib.EINVAL and b"negative window" in lib.kvpath_last_error()


def test_unsupported_is_not_implemented(lib) -> None:
    """A valid case no kernel serves (fp8 cache with an fp32 q) is EUNSUPPORTED, which the
    Python layer raises as NotImplementedError (kelpie's refusal convention)."""
    cache = _cache(dtype=_lib.FP8_E4M3, scale=0x4000, stride_page=16 * 2 * 2 * 64)
    q = _lib.Rows(0x2000, 4, 4, 64, 256, 64, _lib.F32)
    out = _lib.Rows(0x3000, 4, 4, 64, 256, 64, _lib.F32)
    plan = _lib.Plan(0x10, 0x20, 0x30, 0x40, 0x50, 4, 2, 3, 3)
    opts = _lib.AttnOpts(0, None, 1, 512)
    ws = lib.kvpath_workspace_bytes(4, 2, 4, 2, 64, 3, 16, 512)
    st = lib.kvpath_attend(ctypes.byref(q), ctypes.byref(cache), ctypes.byref(plan),
                           ctypes.byref(opts), ctypes.byref(out), 0x10000, ws, None)
    assert st == _lib.EUNSUPPORTED
    with pytest.raises(NotImplementedError):
        _lib.check("attend", st)


def test_python_layer_refuses_cpu_tensors() -> None:
    """There is no CPU path: CPU tensors raise instead of computing."""
    from workloads import Batch, step_args

    args = step_args(Batch(entries=((3, 1),), tokens=1, reqs=1, heads=4, kv_heads=2,
                           head_dim=32, block=4), "cpu", torch.bfloat16)
    with pytest.raises(RuntimeError, match="no CPU path"):
        kvpath.paged_attention(*args)
    with pytest.raises(RuntimeError, match="no CPU path"):
        kvpath.write_kv(args[3], args[1], args[2], args[9])


def test_newest_positions_assert() -> None:
    """kvpath.assert_newest_positions (kelpie's own device assert, for callers that want it)
    accepts the sample plans and refuses a plan whose row sits at a wrong position, as kelpie's
    _assert_newest_positions does (on CPU tensors torch._assert_async raises at once)."""
    from workloads import Batch, step_args

    batch = Batch(entries=((16, 1), (63, 4), (5, 16)), tokens=24, reqs=4, heads=8, kv_heads=2,
                  head_dim=32, block=16)
    args = step_args(batch, "cpu", torch.float32, seed=3)
    rr, pos, qsl, lens = args[4], args[5], args[6], args[7]
    kvpath.assert_newest_positions(rr, pos, qsl, lens)
    bad = pos.clone()
    bad[2] += 1
    with pytest.raises(RuntimeError):
        kvpath.assert_newest_positions(rr, bad, qsl, lens)
    pad = pos.clone()
    pad[-1] = 12345  # pad rows are not checked
    kvpath.assert_newest_positions(rr, pad, qsl, lens)


def test_split_choice_properties(lib) -> None:
    """Over a seeded sweep of step shapes: the floor length is a multiple of 32 of at least 512
    keys; the slots are at least one, no more than the table could fill at the floor, and do not
    grow with the table's width once it exceeds that (kelpie pads tables to max_seq_len), but for
    a table of at most 768 keys, where a decode step takes one slot; the
    workspace is exactly the slots' partials."""
    g = torch.Generator().manual_seed(5)
    out = _lib.Split()
    for _ in range(400):
        T = int(torch.randint(1, 9000, (1,), generator=g))
        R = int(torch.randint(1, min(T, 512) + 1, (1,), generator=g))
        hkv = [1, 2, 4, 8][int(torch.randint(4, (1,), generator=g))]
        H = hkv * [1, 2, 4, 8][int(torch.randint(4, (1,), generator=g))]
        block = [16, 32, 64][int(torch.randint(3, (1,), generator=g))]
        width = int(torch.randint(1, 9000, (1,), generator=g))
        shape = (T, R, H, hkv, width, block)
        assert lib.kvpath_split_plan(*shape, 0, ctypes.byref(out)) == _lib.OK
        part, slots = out.partition_tokens, out.slots
        assert out.per_entry == 1 and part % 32 == 0 and part >= 512, shape
        assert 1 <= slots <= max(1, -(-width * block // part)), shape
        assert lib.kvpath_split_plan(T, R, H, hkv, width * 64, block, 0, ctypes.byref(out)) == 0
        # (A step over at most 768 keys may take one slot: decode's one partition per entry.)
        assert out.slots >= slots and (slots == -(-width * block // part) or out.slots == slots
                                       or (slots == 1 and width * block <= 768))
        for dim in (64, 128):
            rows = T * H * slots
            want = (rows * dim * 4 + 255) // 256 * 256 + rows * 8
            assert lib.kvpath_workspace_bytes(T, R, H, hkv, dim, width, block, 0) == want, shape


def test_workspace_bound_covers_every_smaller_step(lib) -> None:
    """kvpath_workspace_bytes is per exact shape: at a 128k-key table (H 32 / Hkv 8 / D 128) a
    five-entry decode step needs more than a six-, seven- or eight-entry one, because the split
    gives more entries fewer slots each. kvpath_workspace_bytes_max(max_T, max_R, ...) is at
    least kvpath_workspace_bytes of every step with T <= max_T rows and R <= max_R entries
    (checked exhaustively on small bounds, by a seeded sample on large ones), and never shrinks
    as either bound grows."""
    exact = lib.kvpath_workspace_bytes
    bound = lib.kvpath_workspace_bytes_max
    shape = (32, 8, 128, 8192, 16, 0)  # H, Hkv, D, width (128k keys), block, partition
    assert exact(5, 5, *shape) > exact(8, 8, *shape)  # the non-monotone case
    assert bound(8, 8, *shape) >= max(exact(t, r, *shape) for t in range(1, 9) for r in range(1, 9))
    for dims in ((32, 8, 128, 8192, 16, 0), (64, 8, 64, 64, 16, 0), (32, 8, 128, 300, 16, 0),
                 (16, 1, 64, 2048, 32, 0), (32, 8, 128, 8192, 16, 512)):
        for max_t, max_r in ((1, 1), (4, 4), (16, 8), (40, 3), (64, 64), (300, 16)):
            b = bound(max_t, max_r, *dims)
            worst = max(exact(t, r, *dims) for t in range(1, max_t + 1) for r in range(1, max_r + 1))
            assert b >= worst, (dims, max_t, max_r, b, worst)
            assert b == max(b, exact(max_t, max_r, *dims))
    g = torch.Generator().manual_seed(9)
    for _ in range(40):
        max_t = int(torch.randint(1, 4096, (1,), generator=g))
        max_r = int(torch.randint(1, 257, (1,), generator=g))
        b = bound(max_t, max_r, *shape)
        for _ in range(50):
            t = int(torch.randint(1, max_t + 1, (1,), generator=g))
            r = int(torch.randint(1, max_r + 1, (1,), generator=g))
            assert exact(t, r, *shape) <= b, (t, r, max_t, max_r)
    prev = 0
    for max_t in range(1, 200):
        b = bound(max_t, 64, *shape)
        assert b >= prev, max_t
        prev = b
    prev = 0
    for max_r in range(1, 200):
        b = bound(256, max_r, *shape)
        assert b >= prev, max_r
        prev = b
    assert bound(-1, 4, *shape) == -1 and bound(4, 4, 30, 8, 128, 64, 16, 0) == -1
    assert kvpath.workspace_bytes_max(64, 64, 32, 8, 128, 8192, 16) == bound(64, 64, *shape)


def test_plan_lengths_are_checked() -> None:
    """The plan's tensors reach the kernels as bare pointers, so one of another length than the
    contract's (row_request, positions, slot_mapping i32[T]; query_start_loc i32[R+1]; block_table
    i32[R, P]) is refused on the host, before anything reads past its end."""
    import importlib

    from workloads import Batch, step_args

    pa = importlib.import_module("kvpath.paged_attention")  # the module (kvpath.paged_attention is the op)
    batch = Batch(entries=((16, 1), (63, 4), (5, 16)), tokens=24, reqs=4, heads=8, kv_heads=2,
                  head_dim=32, block=16)
    args = step_args(batch, "cpu", torch.float32, seed=3)
    rr, pos, qsl, lens, table, slots = (args[i] for i in (4, 5, 6, 7, 8, 9))
    T = rr.shape[0]
    pa._plan(rr, qsl, lens, table, slots, T, pos)  # the valid plan
    cases = {
        "row_request": (rr[:-1], qsl, lens, table, slots, pos),
        "positions": (rr, qsl, lens, table, slots, pos[:-1]),
        "slot_mapping": (rr, qsl, lens, table, slots[:-1], pos),
        "query_start_loc": (rr, qsl[:-1], lens, table, slots, pos),
        "block_table": (rr, qsl, lens, table[:-1], slots, pos),
    }
    for what, (a, b, c, d, e, f) in cases.items():
        with pytest.raises(ValueError, match=what):
            pa._plan(a, b, c, d, e, T, f)
