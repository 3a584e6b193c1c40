"""GPU parity: the HIP path through the C ABI against the CPU oracle on the same seeded inputs.

Byte work (append, gather, copy_blocks, fp8 quantize-on-append) is compared bit for bit, every
page but the null page 0 (pad rows all write its scratch slot). Attention is graded as the
reference grades it (kelpie bench/correctness.py:28-51: within max(2 x the bf16 reference's own
error, 2e-2 x max|truth|) of the fp64 truth) AND against the fixed tolerance of this build:
|out - truth| <= 2e-2 + 1e-2 |truth| for bf16, 5e-2 + 1e-2 |truth| for an fp8 cache; pad rows
exactly zero.
"""

from __future__ import annotations

import dataclasses

import pytest
import torch

import kvpath
from gpu_support import compact_cpu, dequantized
from helpers import digest, golden_args, golden_batch, within
from workloads import Batch, config_batch, copy_pairs, step_args, synthetic
from oracle import attention as oracle
from oracle import kvbytes

pytestmark = pytest.mark.gpu

BF16_ATOL, BF16_RTOL = 2e-2, 1e-2
FP8_ATOL, FP8_RTOL = 5e-2, 1e-2


def say(*parts) -> None:
    print("[gpu]", *parts, flush=True)


def _engine_member(pages: int, block: int, heads: int, dim: int, dtype, device="cuda",
                   members: int = 2) -> torch.Tensor:
    arena = torch.zeros(pages, block, members, 2, heads, dim, dtype=dtype, device=device)
    return arena[:, :, members - 1].permute(0, 2, 1, 3, 4)


def _random_fill(member: torch.Tensor, seed: int) -> None:
    g = torch.Generator(device=member.device).manual_seed(seed)
    member.copy_(torch.randn(member.shape, generator=g, device=member.device).to(member.dtype))


# ---- append / gather / copy_blocks: bit-exact ---------------------------------------------------


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows", [1, 7, 64, 4096])
def test_append_bit_exact(dtype, rows) -> None:
    say("append", dtype, rows)
    pages, block, heads, dim = 512, 16, 8, 128
    kv = _engine_member(pages, block, heads, dim, dtype)
    _random_fill(kv, 1)
    g = torch.Generator().manual_seed(rows)
    slots = (torch.randperm(pages * block - block, generator=g)[:rows] + block).to(torch.int32)
    k = torch.randn(rows, heads, dim, generator=g).to(dtype)
    v = torch.randn(rows, heads, dim, generator=g).to(dtype)
    want = compact_member(kv)
    kvbytes.kv_append(want, k, v, slots)
    kvpath.write_kv(kv, k.cuda(), v.cuda(), slots.cuda())
    torch.cuda.synchronize()
    got = compact_member(kv)
    assert torch.equal(got.contiguous().view(torch.uint8), want.contiguous().view(torch.uint8))


@pytest.mark.parametrize("heads,dim,dtype", [
    (4, 128, torch.bfloat16),   # 1 KiB per member: one chunk per lane
    (8, 256, torch.float32),    # 8 KiB per member
    (1, 128, torch.bfloat16),   # 256 B per member: any-size 16-byte chunk path
    (3, 64, torch.float16),     # 384 B per member
    (2, 40, torch.bfloat16),    # 160 B per member: not whole 64-lane rows
])
def test_append_row_shapes(heads, dim, dtype) -> None:
    """Every append path (whole-row waves, any-size 16-byte chunks) at an odd row count."""
    say("append shape", heads, dim, dtype)
    pages, block, rows = 64, 16, 37
    kv = _engine_member(pages, block, heads, dim, dtype)
    _random_fill(kv, 5)
    g = torch.Generator().manual_seed(heads * 1000 + dim)
    slots = (torch.randperm(pages * block - block, generator=g)[:rows] + block).to(torch.int32)
    slots[5] = -1  # out of the pool: skipped
    k = torch.randn(rows, heads, dim, generator=g).to(dtype)
    v = torch.randn(rows, heads, dim, generator=g).to(dtype)
    want = compact_member(kv)
    keep = slots >= 0
    kvbytes.kv_append(want, k[keep], v[keep], slots[keep])
    kvpath.write_kv(kv, k.cuda(), v.cuda(), slots.cuda())
    torch.cuda.synchronize()
    got = compact_member(kv)
    assert torch.equal(got.contiguous().view(torch.uint8), want.contiguous().view(torch.uint8))


def test_append_converts_like_torch() -> None:
    """An fp32 step into a bf16 cache: the stored bytes are torch's round-to-nearest-even cast."""
    say("append f32->bf16")
    kv = _engine_member(64, 16, 8, 128, torch.bfloat16)
    g = torch.Generator().manual_seed(2)
    k = torch.randn(33, 8, 128, generator=g) * 3
    v = torch.randn(33, 8, 128, generator=g) * 3
    slots = (torch.randperm(63 * 16, generator=g)[:33] + 16).to(torch.int32)
    kvpath.write_kv(kv, k.cuda(), v.cuda(), slots.cuda())
    ref = _engine_member(64, 16, 8, 128, torch.bfloat16, "cpu")
    oracle.write_kv(ref, k, v, slots)
    assert torch.equal(kv.cpu().view(torch.int16), ref.view(torch.int16))


def test_append_pad_rows_hit_only_the_scratch_slot() -> None:
    """Pad rows all target page 0's last row; every other page is written only by real rows."""
    say("append pads")
    kv = _engine_member(32, 16, 8, 128, torch.bfloat16)
    _random_fill(kv, 3)
    before = kv.cpu().clone()
    g = torch.Generator().manual_seed(4)
    slots = torch.tensor([16 * 5 + 3, 16 * 9, 15, 15, 15], dtype=torch.int32)
    k = torch.randn(5, 8, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(5, 8, 128, generator=g).to(torch.bfloat16)
    kvpath.write_kv(kv, k.cuda(), v.cuda(), slots.cuda())
    after = kv.cpu()
    assert torch.equal(after[1:5].view(torch.int16), before[1:5].view(torch.int16))
    assert torch.equal(after[5, 0, 3].view(torch.int16), k[0].view(torch.int16))
    assert torch.equal(after[9, 1, 0].view(torch.int16), v[1].view(torch.int16))
    assert torch.equal(after[0, :, :15].view(torch.int16), before[0, :, :15].view(torch.int16))


def test_gather_bit_exact() -> None:
    say("gather")
    batch = Batch(entries=((100, 1), (37, 1), (5, 1)), tokens=4, reqs=4, heads=32, kv_heads=8,
                  head_dim=128, block=16, sinks=False)
    args = step_args(batch, "cuda", torch.bfloat16, seed=3)
    kv_member, table = args[3], args[8]
    gk, gv = kvpath.kv_gather(kv_member, table)
    wk, wv = kvbytes.kv_gather(compact_member(kv_member), table.cpu(), table.shape[1])
    assert torch.equal(gk.cpu().view(torch.int16), wk.view(torch.int16))
    assert torch.equal(gv.cpu().view(torch.int16), wv.view(torch.int16))


@pytest.mark.parametrize("dtype,heads,dim", [(torch.float32, 4, 128),
                                             (torch.float8_e4m3fn, 8, 128),
                                             (torch.bfloat16, 2, 64)])
def test_gather_dtypes_strides_and_bad_ids(dtype, heads, dim) -> None:
    """Gather from f32, fp8 and bf16 members, through a block table that is a column slice of a
    wider one (row stride > width), with a null page, a page id past the pool and a negative id
    in it: bit-exact against the oracle; an id outside the pool gives zeros."""
    say("gather", dtype, heads, dim)
    pages, block = 96, 16
    member = _engine_member(pages, block, heads, dim,
                            torch.uint8 if dtype == torch.float8_e4m3fn else dtype)
    if dtype == torch.float8_e4m3fn:
        g = torch.Generator().manual_seed(4)
        member.copy_(torch.randint(0, 126, member.shape, generator=g, dtype=torch.uint8).cuda())
        member = member.view(torch.float8_e4m3fn)
    else:
        _random_fill(member, 4)
    g = torch.Generator().manual_seed(5)
    wide = torch.randint(1, pages, (5, 40), generator=g, dtype=torch.int32)
    wide[0, 3] = 0            # the null page
    wide[1, 0] = pages + 3    # past the pool
    wide[2, 5] = -7           # negative
    table = wide.cuda()[:, :12]  # row stride 40, width 12
    assert table.stride(0) == 40
    gk, gv = kvpath.kv_gather(member, table)
    ref = compact_member(member)
    wk, wv = kvbytes.kv_gather(ref, table.cpu(), 12)
    bits = torch.uint8 if dtype == torch.float8_e4m3fn else (
        torch.int32 if dtype == torch.float32 else torch.int16)
    assert torch.equal(gk.cpu().view(bits), wk.view(bits))
    assert torch.equal(gv.cpu().view(bits), wv.view(bits))
    assert not bool(gk[1, :block].cpu().view(bits).any())  # the page past the pool: zeros
    assert not bool(gv[2, 5 * block:6 * block].cpu().view(bits).any())


def compact_member(kv_member: torch.Tensor) -> torch.Tensor:
    """The whole member on the CPU, in a fresh arena-layout view."""
    pages, _, block, heads, dim = kv_member.shape
    out = _engine_member(pages, block, heads, dim, kv_member.dtype, "cpu", members=1)
    out.copy_(kv_member.cpu())
    return out


@pytest.mark.parametrize("dtype,heads,dim,block", [
    (torch.bfloat16, 8, 128, 16),       # 2 KiB rows per member: whole rows per wave
    (torch.float8_e4m3fn, 8, 128, 16),  # 1 KiB rows, with the fp8 scales
    (torch.float32, 8, 128, 16),        # 4 KiB rows
    (torch.bfloat16, 4, 128, 32),       # 1 KiB rows, 32-row pages
    (torch.bfloat16, 1, 128, 16),       # 256 B rows: any-size 16-byte chunk path
    (torch.float16, 3, 40, 16),         # 240 B rows
])
def test_copy_blocks_bit_exact(dtype, heads, dim, block) -> None:
    say("copy_blocks", dtype, heads, dim, block)
    pages = 300
    scale = None
    if dtype == torch.float8_e4m3fn:
        kv = _engine_member(pages, block, heads, dim, torch.uint8).view(torch.float8_e4m3fn)
        kv.view(torch.uint8).copy_(torch.randint(0, 126, kv.shape, dtype=torch.uint8, device="cuda"))
        scale = torch.rand(pages, 2, heads, device="cuda")
    else:
        kv = _engine_member(pages, block, heads, dim, dtype)
        _random_fill(kv, 5)
    g = torch.Generator().manual_seed(6)
    perm = torch.randperm(pages - 1, generator=g) + 1
    src, dst = perm[:100].to(torch.int32), perm[100:200].to(torch.int32)
    src[7] = -1  # out of the pool: the pair is skipped
    want = compact_member(kv)
    want_scale = scale.cpu().clone() if scale is not None else None
    keep = src >= 0
    kvbytes.copy_blocks(want, src[keep], dst[keep], want_scale)
    kvpath.copy_blocks(kv, src.cuda(), dst.cuda(), scale)
    torch.cuda.synchronize()
    assert torch.equal(compact_member(kv).contiguous().view(torch.uint8),
                       want.contiguous().view(torch.uint8))
    if scale is not None:
        assert torch.equal(scale.cpu(), want_scale)


# ---- fp8 quantize-on-append: bytes and scales bit-exact ---------------------------------------------


@pytest.mark.parametrize("dim,in_dtype", [(128, torch.bfloat16), (64, torch.bfloat16),
                                          (256, torch.bfloat16), (128, torch.float32)])
def test_fp8_append_bit_exact_over_steps(dim, in_dtype) -> None:
    """A prefill chunk, then decode steps and a multi-row step, into an fp8 member with stale
    scales and bytes: every page's bytes and scales equal the C oracle's after each step (bf16
    rows at D 64/128/256 take the run kernel, f32 rows the generic one)."""
    say("fp8 append steps", dim, in_dtype)
    pages, block, heads = 40, 16, 8
    kv = _engine_member(pages, block, heads, dim, torch.uint8).view(torch.float8_e4m3fn)
    g = torch.Generator().manual_seed(7)
    kv.view(torch.uint8).copy_(torch.randint(0, 120, kv.shape, generator=g, dtype=torch.uint8).cuda())
    scale = (torch.rand(pages, 2, heads, generator=g) * 0.05).cuda()  # stale owners' scales
    ref_kv = compact_member(kv)
    ref_scale = scale.cpu().clone()
    order = (torch.randperm(pages - 1, generator=g) + 1).tolist()
    table = torch.tensor([order[:10], order[10:20], order[20:30]], dtype=torch.int32)
    lens = [0, 0, 0]

    def step(rows: list[int]) -> None:
        slots = []
        for r, n in enumerate(rows):
            for i in range(n):
                p = lens[r] + i
                slots.append(int(table[r, p // block]) * block + p % block)
            lens[r] += n
        t = len(slots)
        x = torch.randn(t, heads, dim, generator=g)
        x = torch.where(torch.rand(t, heads, dim, generator=g) < 0.01, x * 20, x)
        k = x.to(torch.bfloat16).to(in_dtype)
        v = (torch.randn(t, heads, dim, generator=g) * (1 + lens[0] % 3)).to(in_dtype)
        s = torch.tensor(slots, dtype=torch.int32)
        kvbytes.kv_append_fp8(ref_kv, ref_scale, k, v, s)
        kvpath.write_kv(kv, k.cuda(), v.cuda(), s.cuda(), scale)
        torch.cuda.synchronize()
        assert torch.equal(compact_member(kv)[1:].contiguous().view(torch.uint8),
                           ref_kv[1:].contiguous().view(torch.uint8)), rows
        assert torch.equal(scale.cpu()[1:], ref_scale[1:]), rows

    step([37, 5, 16])     # prefill: fresh pages, partial and full
    for _ in range(12):
        step([1, 1, 1])   # decode: scale growth + requantization
    step([4, 0, 20])      # multi-row step across a page boundary


@pytest.mark.parametrize("offset,dim", [(0, 128), (5, 128), (0, 64)])
def test_fp8_append_prefill_sized_bit_exact(offset, dim) -> None:
    """Prefill-sized fp8 appends (34,000 rows: the run kernel's 16-row chunks) starting at a page
    boundary or mid-page (runs then straddle the chunks), at D 128 and 64, with stale bytes and
    scales, and a last row whose slot lies outside the pool: bytes and scales equal the C
    oracle's. (A step's rows that share a page are consecutive, as in every kelpie plan.)"""
    say("fp8 append prefill-sized, offset", offset, "dim", dim)
    pages, block, heads = 2400, 16, 8
    kv = _engine_member(pages, block, heads, dim, torch.uint8).view(torch.float8_e4m3fn)
    g = torch.Generator().manual_seed(11 + offset)
    kv.view(torch.uint8).copy_(torch.randint(0, 120, kv.shape, generator=g, dtype=torch.uint8).cuda())
    scale = (torch.rand(pages, 2, heads, generator=g) * 0.05).cuda()
    ref_kv = compact_member(kv)
    ref_scale = scale.cpu().clone()
    rows = 34000
    order = (torch.randperm(pages - 1, generator=g) + 1)
    pos = torch.arange(offset, offset + rows)
    slots = (order[pos // block] * block + pos % block).to(torch.int32)
    slots[-1] = pages * block + 7  # outside the pool (last, as pad rows come): skipped
    x = torch.randn(rows, heads, dim, generator=g)
    k = torch.where(torch.rand(rows, heads, dim, generator=g) < 0.01, x * 20, x).to(torch.bfloat16)
    v = torch.randn(rows, heads, dim, generator=g).to(torch.bfloat16)
    kvbytes.kv_append_fp8(ref_kv, ref_scale, k, v, slots)
    kvpath.write_kv(kv, k.cuda(), v.cuda(), slots.cuda(), scale)
    torch.cuda.synchronize()
    assert torch.equal(compact_member(kv)[1:].contiguous().view(torch.uint8),
                       ref_kv[1:].contiguous().view(torch.uint8))
    assert torch.equal(scale.cpu()[1:], ref_scale[1:])


@pytest.mark.parametrize("rows", [48, 34000])
def test_fp8_append_non_finite_rows_bit_exact(rows) -> None:
    """Rows holding +-inf or NaN in some (member, head) runs, among finite ones, in decode-sized
    and prefill-sized steps: the run kernel takes such a run through the f32 absmax (NaN skipped)
    and the clamped conversion, the rest through its finite path, and an inf scale stores zeros;
    then a second step appends a row after each decode row, an inf among them growing a finite
    scale (the requantization's shift runs to the overflow). Bytes and scale bits equal the C
    oracle's after each step."""
    say("fp8 append non-finite rows", rows)
    pages, block, heads, dim = 2400, 16, 8, 128
    kv = _engine_member(pages, block, heads, dim, torch.uint8).view(torch.float8_e4m3fn)
    g = torch.Generator().manual_seed(29)
    kv.view(torch.uint8).copy_(torch.randint(0, 120, kv.shape, generator=g, dtype=torch.uint8).cuda())
    scale = (torch.rand(pages, 2, heads, generator=g) * 0.05).cuda()
    ref_kv = compact_member(kv)
    ref_scale = scale.cpu().clone()
    order = (torch.randperm(pages - 1, generator=g) + 1)
    pos = torch.arange(rows) * (1 if rows > 1000 else 16)  # decode-sized: one row per page
    slots = (order[pos // block] * block + pos % block).to(torch.int32)
    k = torch.randn(rows, heads, dim, generator=g)
    v = torch.randn(rows, heads, dim, generator=g)
    k[3, 2, 5] = float("inf")
    k[7, 0, 100] = float("-inf")
    v[3, 5, 9] = float("nan")
    k[40, 1, 0] = float("nan")
    v[41, 7, 127] = float("inf")

    def step(k: torch.Tensor, v: torch.Tensor, slots: torch.Tensor) -> None:
        k, v = k.to(torch.bfloat16), v.to(torch.bfloat16)
        kvbytes.kv_append_fp8(ref_kv, ref_scale, k, v, slots)
        kvpath.write_kv(kv, k.cuda(), v.cuda(), slots.cuda(), scale)
        torch.cuda.synchronize()
        assert torch.equal(compact_member(kv)[1:].contiguous().view(torch.uint8),
                           ref_kv[1:].contiguous().view(torch.uint8))
        assert torch.equal(scale.cpu()[1:].view(torch.int32), ref_scale[1:].view(torch.int32))

    step(k, v, slots)
    if rows < 1000:
        k2 = torch.randn(rows, heads, dim, generator=g)
        v2 = torch.randn(rows, heads, dim, generator=g)
        k2[10, 4, 7] = float("inf")
        v2[11, 2, 2] = float("nan")
        step(k2, v2, slots + 1)


# ---- attention: golden cases and the configurations ---------------------------------------------------


GOLDEN_CASES = ["sample_batch", "c1_tiny_decode", "decode_padded", "decode_window",
                "verify_ragged", "drafter", "prefill_mixed", "llama_verify"]


@pytest.mark.parametrize("name", GOLDEN_CASES)
def test_golden_cases_bf16(name, golden) -> None:
    """The reference's own cases, bf16: within its error budget of its fp64 truth, within the
    fixed tolerance, pad rows exactly 0, and the pool after append byte-identical to the
    reference's."""
    meta, arrays = golden
    say("golden", name)
    batch = golden_batch(name, meta)
    args = golden_args(name, golden, "cuda", torch.bfloat16)
    out = kvpath.paged_attention(*args)
    torch.cuda.synchronize()
    truth = torch.from_numpy(arrays[f"{name}/out_float64"]).double()
    ref = torch.from_numpy(arrays[f"{name}/out_bfloat16"]).view(torch.bfloat16)
    budget = oracle.error_budget(truth, ref)
    err = (out.double().cpu() - truth).abs().max().item()
    assert err <= budget, (name, err, budget)
    ok, ratio = within(out, truth, BF16_ATOL, BF16_RTOL)
    assert ok, (name, ratio)
    n = batch.n_rows
    assert torch.equal(out[n:].cpu(), torch.zeros_like(out[n:].cpu()))
    # The pool after the append equals the oracle's (whose pool digest is the reference's, pinned
    # on the CPU), byte for byte, except the scratch row of page 0 that all pad rows race on.
    cpu_args = golden_args(name, golden, "cpu", torch.bfloat16)
    oracle.write_kv(cpu_args[3], cpu_args[1], cpu_args[2], cpu_args[9])
    got, want = _arena_of(args[3]), _arena_of(cpu_args[3])
    assert torch.equal(got[1:], want[1:]), name
    assert torch.equal(got[0, : batch.block - 1], want[0, : batch.block - 1]), name
    if batch.n_rows == batch.tokens:  # no pad rows: the whole arena is the reference's
        assert digest(got) == meta[name]["pool_after_bf16"], name


def _arena_of(member: torch.Tensor) -> torch.Tensor:
    """The whole arena a two-member step's member views, on the CPU, as [pages, block, 2, 2, Hkv,
    D] raw 16-bit words."""
    pages, _, block, heads, dim = member.shape
    words = torch.empty(0, dtype=torch.int16, device=member.device).set_(member.untyped_storage())
    return words.cpu().reshape(pages, block, 2, 2, heads, dim)


@pytest.mark.parametrize("name", ["sample_batch", "c1_tiny_decode"])
def test_golden_cases_fp32(name, golden) -> None:
    """fp32 inputs (the generic VALU kernel): within the reference's fp32 budget of the truth."""
    meta, arrays = golden
    say("golden fp32", name)
    args = golden_args(name, golden, "cuda", torch.float32)
    out = kvpath.paged_attention(*args)
    truth = torch.from_numpy(arrays[f"{name}/out_float64"]).double()
    ref = torch.from_numpy(arrays[f"{name}/out_float32"])
    budget = oracle.error_budget(truth, ref)
    err = (out.double().cpu() - truth).abs().max().item()
    assert err <= max(budget, 1e-5), (name, err, budget)


def _check_against_oracle(out: torch.Tensor, args_gpu: tuple, entries: list[int] | None,
                          atol: float, rtol: float, kv_scale=None, label="") -> float:
    """Compare `out` (rows of the op on args_gpu, AFTER its append) with the fp64 oracle on the
    same entries. The pool already holds this step's rows, so the oracle attends only."""
    cpu, rows, scale = compact_cpu(args_gpu, entries, kv_scale)
    (q, _, _, member, rr, pos, qsl, lens, table, _, window, sinks, causal) = cpu
    if scale is not None:
        member64 = dequantized(member, scale)
    else:
        member64 = member
    q64, member64 = oracle.upcast((q, member64))
    truth = oracle.attend(q64, member64, rr, pos, qsl, lens, table, window, sinks.double(), causal)
    got = out.cpu()[rows]
    ok, ratio = within(got, truth, atol, rtol)
    say(label, "worst err / tol =", round(ratio, 4))
    assert ok, (label, ratio)
    return ratio


@pytest.mark.parametrize("cfg", [1, 2, 3, 4, 5, 6, 7, 8, 9, 10])
def test_config_attention(cfg) -> None:
    """Each BASELINE configuration (1-5), each workload of the callers next to the path
    (6 chunked prefill, 7/8 gpt-oss full and sliding-window decode with sinks, 9 the DFlash
    drafter's non-causal block), and config 2 at 4096 keys (10), at its real shape (pool,
    heads, context lengths) through the whole op, checked against the fp64 oracle on every
    entry (config 4's in chunks of 16: its pages dequantized to fp64 are ~10 GB at once)."""
    batch, extra = config_batch(cfg)
    say("config", cfg, "entries", len(batch.entries))
    step = synthetic(batch, "cuda", extra["dtype"], seed=cfg, pool_pages=extra["pool_pages"],
                     outliers=extra.get("outliers", 0.0), cache_dtype=extra.get("cache_dtype"))
    args = step.args
    if step.kv_scale is not None:
        out = kvpath.paged_attention_fp8(*args, step.kv_scale)
        atol, rtol = FP8_ATOL, FP8_RTOL
    else:
        out = kvpath.paged_attention(*args)
        atol, rtol = (BF16_ATOL, BF16_RTOL) if extra["dtype"] == torch.bfloat16 else (1e-4, 1e-4)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    # Every entry of every configuration; config 4's sixteen at a time.
    if cfg == 4:
        for lo in range(0, len(batch.entries), 16):
            entries = list(range(lo, min(lo + 16, len(batch.entries))))
            _check_against_oracle(out, args, entries, atol, rtol, step.kv_scale, f"config {cfg} entries {lo}+")
    else:
        _check_against_oracle(out, args, None, atol, rtol, step.kv_scale, f"config {cfg}")


@pytest.mark.parametrize("n,heads,dim,cache", [
    (1, 32, 128, torch.bfloat16),
    (8, 64, 64, torch.bfloat16),      # gpt-oss: 64 q / 8 kv heads, D 64, sinks
    (32, 32, 128, torch.bfloat16),
    (16, 32, 128, torch.float8_e4m3fn),
])
def test_short_decode_tables_take_one_partition(n, heads, dim, cache) -> None:
    """A decode step over a table of at most 768 keys takes one slot: each entry is one
    partition, written to `out` with no reduce. Its output meets the oracle's tolerance and
    agrees with the same step forced through split-KV partitions of 128 keys and the reduce
    (fp32 rounding apart); pad rows stay zero."""
    say("short decode table", n, heads, dim, cache)
    ctx = [int(x) for x in torch.randint(1, 720, (n,), generator=torch.Generator().manual_seed(n))]
    batch = Batch(entries=tuple((c, 1) for c in ctx), tokens=n + 2, reqs=n + 1, heads=heads,
                  kv_heads=8, head_dim=dim, block=16, sinks=heads == 64)
    step = synthetic(batch, "cuda", torch.bfloat16, seed=60 + n, pool_pages=4096,
                     cache_dtype=None if cache == torch.bfloat16 else cache)
    width = step.args[8].shape[1]
    assert width * 16 <= 768
    assert kvpath.split_plan(batch.tokens, batch.reqs, heads, 8, width, 16, 0)[1] == 1
    fp8 = step.kv_scale is not None
    run = ((lambda **kw: kvpath.paged_attention_fp8(*step.args, step.kv_scale, **kw)) if fp8
           else (lambda **kw: kvpath.paged_attention(*step.args, **kw)))
    one = run()
    split = run(partition=128)
    torch.cuda.synchronize()
    assert torch.equal(one[batch.n_rows:].cpu(), torch.zeros_like(one[batch.n_rows:].cpu()))
    atol, rtol = (FP8_ATOL, FP8_RTOL) if fp8 else (BF16_ATOL, BF16_RTOL)
    ok, ratio = within(one.cpu().float(), split.cpu().float(), atol, rtol)
    assert ok, ratio
    _check_against_oracle(one, step.args, None, atol, rtol, step.kv_scale, label="one partition")


def test_config2_padded_to_its_bucket() -> None:
    """BASELINE config 2 as kelpie pads a step to its bucket (c_api.zig:1085-1153): 61 real decode
    entries padded to R = 64, three pad rows, through the whole op (the decode kernel with the
    append fused in). Pad rows are exactly zero; the pool changes only at the real rows' slots
    (and at most the scratch slot, page 0's last row, that pad rows target), holding their k/v
    bit for bit; the real rows match the fp64 oracle."""
    batch, extra = config_batch(2)
    padded = dataclasses.replace(batch, entries=batch.entries[:61])
    assert (padded.tokens, padded.reqs, padded.n_rows) == (64, 64, 61)
    say("config 2 padded to its bucket")
    step = synthetic(padded, "cuda", torch.bfloat16, seed=2, pool_pages=extra["pool_pages"])
    q, k, v, member, rr, pos, qsl, lens, table, slot_map, window, sinks, causal = step.args
    before = member.clone()
    out = kvpath.paged_attention(*step.args)
    torch.cuda.synchronize()
    n, block = padded.n_rows, padded.block
    assert torch.equal(out[n:].cpu(), torch.zeros_like(out[n:].cpu()))
    changed = (member.view(torch.int16) != before.view(torch.int16)).flatten(3).any(3).any(1)
    allowed = torch.zeros_like(changed)
    real = slot_map[:n].long()
    allowed.view(-1)[real] = True
    allowed[0, block - 1] = True
    assert not (changed & ~allowed).any()
    pages, rows = real // block, real % block
    assert torch.equal(member[pages, 0, rows].view(torch.int16), k[:n].view(torch.int16))
    assert torch.equal(member[pages, 1, rows].view(torch.int16), v[:n].view(torch.int16))
    del before
    _check_against_oracle(out, step.args, [0, 30, 60], BF16_ATOL, BF16_RTOL, None, "config 2 padded")


@pytest.mark.parametrize("dim,rows,window,sinks", [
    (128, 1, 0, False),    # decode
    (128, 5, 0, True),     # multi-row (two row tiles), sinks
    (128, 16, 40, False),  # verify-shaped (four row tiles), window
    (64, 1, 0, True),
    (64, 7, 0, False),
    (256, 1, 0, False),
    (256, 3, 24, True),
])
def test_fp8_attention_shapes(dim, rows, window, sinks) -> None:
    """fp8 cache: every tile shape of the fp8 kernels (decode and multi-row, D 64/128/256) with
    contexts that end mid-block and mid-page, against the fp64 oracle on the dequantized pages."""
    say("fp8 shape", dim, rows, window, sinks)
    ctx = [1, 15, 16, 33, 250, 513, 700, 1030]
    batch = Batch(entries=tuple((n, rows) for n in ctx), tokens=len(ctx) * rows + 3,
                  reqs=len(ctx) + 1, heads=16, kv_heads=4, head_dim=dim, block=16,
                  window=window, sinks=sinks)
    step = synthetic(batch, "cuda", torch.bfloat16, seed=dim + rows, pool_pages=512,
                     outliers=0.01, cache_dtype=torch.float8_e4m3fn)
    out = kvpath.paged_attention_fp8(*step.args, step.kv_scale)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    assert torch.equal(out[batch.n_rows:].cpu(), torch.zeros_like(out[batch.n_rows:].cpu()))
    _check_against_oracle(out, step.args, None, FP8_ATOL, FP8_RTOL, step.kv_scale,
                          f"fp8 D{dim} rows{rows}")


def test_partition_size_invariance() -> None:
    """Split-KV is exact up to fp32 rounding: partitions of 32, 96, 160, 512 and 16384 keys agree
    (160 gives an even partition count, the rotated-slot grid)."""
    say("partition invariance")
    batch, extra = config_batch(2)
    batch = Batch(entries=batch.entries[:16], tokens=16, reqs=16, heads=32, kv_heads=8,
                  head_dim=128, block=16, sinks=False)
    step = synthetic(batch, "cuda", torch.bfloat16, seed=11, pool_pages=8192)
    q, k, v, kv_member, rr, pos, qsl, lens, table, slots, window, sinks, causal = step.args
    kvpath.write_kv(kv_member, k, v, slots)
    outs = [kvpath.attend(q, kv_member, rr, qsl, lens, table, window, sinks, causal,
                          partition=p).float() for p in (32, 96, 160, 512, 16384)]
    for o in outs[1:]:
        torch.testing.assert_close(o, outs[0], atol=4e-3, rtol=8e-3)


@pytest.mark.parametrize("cfg", [3, 6])
def test_multi_row_partition_invariance(cfg) -> None:
    """The multi-row kernel's split-KV is exact up to fp32 rounding too: a verify step and a
    chunked-prefill step through the whole op at partitions of 96, 160, 512 and 4096 keys agree."""
    say("multi-row partition invariance", cfg)
    batch, extra = config_batch(cfg)
    batch = Batch(entries=batch.entries[:2], tokens=sum(r for _, r in batch.entries[:2]),
                  reqs=2, heads=batch.heads, kv_heads=batch.kv_heads, head_dim=batch.head_dim,
                  block=batch.block, sinks=batch.sinks)
    outs = []
    for p in (96, 160, 512, 4096):
        step = synthetic(batch, "cuda", torch.bfloat16, seed=21, pool_pages=4096)
        outs.append(kvpath.paged_attention(*step.args, partition=p).float())
    for o in outs[1:]:
        torch.testing.assert_close(o, outs[0], atol=4e-3, rtol=8e-3)


@pytest.mark.parametrize("dim,heads,entries,window,use_sinks,causal", [
    (128, 32, ((0, 100), (37, 64), (700, 129)), 0, False, True),
    (64, 64, ((5, 40), (300, 33), (1000, 70)), 128, True, True),
    (128, 32, ((500, 64), (1200, 80)), 0, False, False),
    (64, 64, ((0, 50), (129, 48)), 37, False, True),
])
def test_prefill_shapes(dim, heads, entries, window, use_sinks, causal) -> None:
    """Prefill-sized steps (16+ row tiles per entry: two tiles per wave) with ragged row counts,
    chunks that start mid-page, windows, sinks and non-causal rows, against the fp64 oracle; at
    the library's partition and at one partition over the whole table, where the kernel writes
    the output itself and zeroes the pad rows (no reduce)."""
    n_rows = sum(r for _, r in entries)
    batch = Batch(entries=entries, tokens=n_rows + 5, reqs=len(entries) + 1, heads=heads,
                  kv_heads=8, head_dim=dim, block=16, window=window, sinks=use_sinks,
                  causal=causal)
    for part in (0, 1 << 16):
        say("prefill shape", dim, heads, entries, window, use_sinks, causal, "partition", part)
        args = step_args(batch, "cuda", torch.bfloat16, seed=dim + n_rows)
        out = kvpath.paged_attention(*args, partition=part)
        torch.cuda.synchronize()
        assert torch.isfinite(out).all()
        assert torch.equal(out[batch.n_rows:].cpu(), torch.zeros_like(out[batch.n_rows:].cpu()))
        _check_against_oracle(out, args, None, BF16_ATOL, BF16_RTOL,
                              label=f"prefill D{dim} partition {part}")


def test_verify_matches_decode_rows() -> None:
    """A verify step's last row sees exactly what a decode row at the same position sees."""
    say("verify vs decode")
    ctx = 700
    verify = Batch(entries=((ctx, 16),), tokens=16, reqs=1, heads=32, kv_heads=8, head_dim=128,
                   block=16, sinks=False)
    args = list(step_args(verify, "cuda", torch.bfloat16, seed=12))
    out_v = kvpath.paged_attention(*args)
    q, _, _, kv_member, rr, pos, qsl, lens, table, slots, window, sinks, causal = args
    # decode-shaped plan for the same entry's last position, pages already written
    d_q = q[15:16].contiguous()
    d_rr = torch.zeros(1, dtype=torch.int32, device="cuda")
    d_qsl = torch.tensor([0, 1], dtype=torch.int32, device="cuda")
    out_d = kvpath.attend(d_q, kv_member, d_rr, d_qsl, lens, table, window, sinks, causal)
    torch.testing.assert_close(out_d.float(), out_v[15:16].float(), atol=4e-3, rtol=8e-3)


@pytest.mark.parametrize("window,use_sinks,causal", [(0, True, True), (128, True, True),
                                                      (37, False, True), (0, False, False)])
def test_window_sinks_causal_variants(window, use_sinks, causal) -> None:
    say("variants", window, use_sinks, causal)
    batch = Batch(entries=((300, 1), (129, 4), (5, 16), (1000, 2)), tokens=24, reqs=5,
                  heads=64, kv_heads=8, head_dim=64, block=16, window=window, sinks=use_sinks,
                  causal=causal)
    args = step_args(batch, "cuda", torch.bfloat16, seed=13)
    out = kvpath.paged_attention(*args)
    _check_against_oracle(out, args, None, BF16_ATOL, BF16_RTOL, label=f"w{window}")
    assert torch.equal(out[batch.n_rows:].cpu(), torch.zeros_like(out[batch.n_rows:].cpu()))


@pytest.mark.parametrize("rows", [1, 16])
def test_window_slid_out_pages_may_be_null(rows) -> None:
    """Sliding-window layers free the pages their window has left (gpt-oss; kelpie nulls them in
    the block table). With every page wholly before each entry's first visible key set to the
    null page 0, the output is unchanged, bit for bit."""
    say("null slid-out pages", rows)
    window = 64
    ctx = [300, 517, 1000, 2047]
    batch = Batch(entries=tuple((n, rows) for n in ctx), tokens=len(ctx) * rows + 2,
                  reqs=len(ctx) + 1, heads=64, kv_heads=8, head_dim=64, block=16, window=window,
                  sinks=True)
    args = list(step_args(batch, "cuda", torch.bfloat16, seed=31))
    q, k, v, kv_member, rr, pos, qsl, lens, table, slots, win, sinks, causal = args
    kvpath.write_kv(kv_member, k, v, slots)
    full = kvpath.attend(q, kv_member, rr, qsl, lens, table, win, sinks, causal)
    nulled = table.clone()
    for r, (n, _) in enumerate(batch.entries):
        first_visible = max(0, n - window + 1)  # the entry's first row (position n) sees from here
        nulled[r, : first_visible // batch.block] = 0
    assert int((nulled == 0).sum()) > int((table == 0).sum())
    out = kvpath.attend(q, kv_member, rr, qsl, lens, nulled, win, sinks, causal)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), full.cpu())


@pytest.mark.parametrize("cfg", [2, 6])
def test_split_entry_points_match_attend(cfg) -> None:
    """The C ABI's two halves, kvpath_attend_partitions then kvpath_attend_reduce, give exactly
    kvpath_attend's output for a decode step (split-KV: both go through the same partials). For a
    prefill step whose single partition kvpath_attend serves with direct output, the halves still
    go through partials, which a bf16 q keeps normalized in bf16: the two outputs are at most one
    extra bf16 rounding apart (the sink term is applied after the partial's rounding)."""
    import ctypes

    from kvpath import _lib
    from kvpath.paged_attention import _cache, _dtype_code, _opts, _plan, _rows, _stream, _workspace

    say("split entry points", cfg)
    batch, _ = config_batch(cfg)
    batch = Batch(entries=batch.entries[:4], tokens=sum(r for _, r in batch.entries[:4]) + 1,
                  reqs=5, heads=batch.heads, kv_heads=batch.kv_heads, head_dim=batch.head_dim,
                  block=batch.block, sinks=True)
    q, k, v, kv_member, rr, pos, qsl, lens, table, slots, window, sinks, causal = step_args(
        batch, "cuda", torch.bfloat16, seed=40 + cfg)
    kvpath.write_kv(kv_member, k, v, slots)
    part = 0  # the library's split of each entry by its own length
    want = kvpath.attend(q, kv_member, rr, qsl, lens, table, window, sinks, causal, partition=part)
    lib = _lib.load()
    cache = _cache(kv_member, None)
    qr, qq = _rows(q, "q")
    plan, keep = _plan(rr, qsl, lens, table, None, q.shape[0])
    opts, sinks32 = _opts(window, sinks, q.shape[1], causal, part)
    ws = _workspace(q.device, q.shape[0], lens.shape[0], q.shape[1], kv_member.shape[3],
                    q.shape[2], table.shape[1], kv_member.shape[2], part)
    got = torch.full_like(want, float("nan"))
    outr = _lib.Rows(got.data_ptr(), q.shape[0], q.shape[1], q.shape[2], got.stride(0),
                     q.shape[2], _dtype_code(got, "out"))
    stream = _stream(q.device)
    _lib.check("attend_partitions", lib.kvpath_attend_partitions(
        ctypes.byref(qr), ctypes.byref(cache), ctypes.byref(plan), ctypes.byref(opts),
        ws.data_ptr(), ws.numel(), stream))
    _lib.check("attend_reduce", lib.kvpath_attend_reduce(
        ctypes.byref(qr), ctypes.byref(cache), ctypes.byref(plan), ctypes.byref(opts),
        ctypes.byref(outr), ws.data_ptr(), ws.numel(), stream))
    torch.cuda.synchronize()
    del qq, keep, sinks32
    if cfg == 2:
        assert torch.equal(got.cpu(), want.cpu())
    else:
        got64, want64 = got.cpu().double(), want.cpu().double()
        assert bool(((got64 - want64).abs() <= 2.0 ** -7 * want64.abs()).all())
        assert not torch.equal(got.cpu(), torch.zeros_like(got.cpu()))


def test_position_checks_pass_valid_plans() -> None:
    """kelpie's own device assert (kvpath.assert_newest_positions, torch._assert_async) passes
    the plan of a decode + verify + pad step on the GPU, and the op's output with the plan
    check's opt-in slot comparison on equals its output without it, with the plan-status word
    clear. (A failing plan is tested on the CPU for the assert, which on the GPU would abort the
    stream, and in test_gpu_plan_check.py for the kernels' check.)"""
    say("position checks")
    batch = Batch(entries=((300, 1), (129, 4), (5, 16), (1000, 2)), tokens=24, reqs=5,
                  heads=32, kv_heads=8, head_dim=128, block=16, sinks=False)
    args = step_args(batch, "cuda", torch.bfloat16, seed=50)
    kvpath.assert_newest_positions(args[4], args[5], args[6], args[7])
    kvpath.clear_plan_status()
    plain = kvpath.paged_attention(*args)
    old = kvpath.set_slot_check(True)
    try:
        checked = kvpath.paged_attention(*step_args(batch, "cuda", torch.bfloat16, seed=50))
    finally:
        kvpath.set_slot_check(old)
    torch.cuda.synchronize()
    assert torch.equal(plain.cpu(), checked.cpu())
    assert kvpath.plan_status() == 0


@pytest.mark.parametrize("window,ctx,cache", [
    (128, (300, 517, 1000, 2047), torch.bfloat16),      # gpt-oss sliding window: one partition
    (0, (1, 15, 100, 480), torch.bfloat16),             # a short table: one partition
    (40, (300, 517, 1000, 2047), torch.float8_e4m3fn),  # fp8 decode, window
])
def test_decode_direct_output(window, ctx, cache) -> None:
    """Decode steps whose keys fit one partition: the decode kernel writes the output itself (no
    reduce) and an extra grid slice zeroes the pad rows. Against the fp64 oracle, and against
    the split path (96-key partitions, reduce) within fp32 rounding."""
    say("decode direct", window, ctx, cache)
    batch = Batch(entries=tuple((n, 1) for n in ctx), tokens=len(ctx) + 3, reqs=len(ctx) + 1,
                  heads=64, kv_heads=8, head_dim=64, block=16, window=window, sinks=True)
    fp8 = cache == torch.float8_e4m3fn
    outs = []
    for part in (0, 96):
        step = synthetic(batch, "cuda", torch.bfloat16, seed=60, pool_pages=1024,
                         cache_dtype=cache if fp8 else None)
        if fp8:
            out = kvpath.paged_attention_fp8(*step.args, step.kv_scale, partition=part)
        else:
            out = kvpath.paged_attention(*step.args, partition=part)
        torch.cuda.synchronize()
        assert torch.equal(out[batch.n_rows:].cpu(), torch.zeros_like(out[batch.n_rows:].cpu()))
        atol, rtol = (FP8_ATOL, FP8_RTOL) if fp8 else (BF16_ATOL, BF16_RTOL)
        _check_against_oracle(out, step.args, None, atol, rtol, step.kv_scale,
                              label=f"decode direct w{window} partition {part}")
        outs.append(out.float())
    torch.testing.assert_close(outs[0], outs[1], atol=4e-3, rtol=8e-3)


def _random_cases(n: int, seed: int) -> list[tuple]:
    g = torch.Generator().manual_seed(seed)

    def pick(options):
        return options[int(torch.randint(len(options), (1,), generator=g))]

    cases = []
    for i in range(n):
        dim = pick([64, 128, 256])
        hkv = pick([1, 2, 4, 8])
        heads = hkv * pick([1, 2, 4, 8])
        rows = pick([1, 1, 2, 5, 16, 40])
        n_entries = 1 + int(torch.randint(6, (1,), generator=g))
        ctx = tuple(int(torch.randint(1500, (1,), generator=g)) for _ in range(n_entries))
        window = pick([0, 0, 17, 128, 700])
        cases.append((i, dim, hkv, heads, rows, ctx, window, pick([True, False]),
                      pick([True, True, False]), pick([0, 0, 64, 96, 416]),
                      pick([torch.bfloat16, torch.bfloat16, torch.float8_e4m3fn]), 16))
    return cases


def _random_page_cases(n: int, seed: int) -> list[tuple]:
    """Like _random_cases, over 16-, 32- and 64-key pages and up to 160 rows per entry (the
    prefill-sized two-tile kernel), same tuple layout."""
    g = torch.Generator().manual_seed(seed)

    def pick(options):
        return options[int(torch.randint(len(options), (1,), generator=g))]

    cases = []
    for i in range(n):
        dim = pick([64, 128, 256])
        hkv = pick([1, 2, 8])
        heads = hkv * pick([1, 4, 8])
        rows = pick([1, 3, 16, 64, 160])
        block = pick([16, 32, 64])
        n_entries = 1 + int(torch.randint(4, (1,), generator=g))
        ctx = tuple(int(torch.randint(1200, (1,), generator=g)) for _ in range(n_entries))
        cases.append((1000 + i, dim, hkv, heads, rows, ctx, pick([0, 0, 100]), pick([True, False]),
                      pick([True, True, False]), pick([0, 0, 96, 512]),
                      pick([torch.bfloat16, torch.bfloat16, torch.float8_e4m3fn]), block))
    return cases


@pytest.mark.parametrize("case", _random_cases(120, seed=77) + _random_page_cases(40, seed=31337),
                         ids=lambda c: f"case{c[0]}")
def test_random_shapes_against_oracle(case) -> None:
    """A seeded sweep over the op's shape space (head dims, GQA ratios, row counts up to 160,
    contexts up to 1.5k, 16- to 64-key pages, windows, sinks, causal or not, partition lengths,
    bf16 or fp8 cache), each step checked against the fp64 oracle with its pad rows exactly
    zero. (1700 further cases of other seeds, run once, also pass, and 2800 of larger shapes:
    contexts to 4096 keys, up to 12 entries, 1-300 rows; a sweep like this is what found the
    D 256 decode fault.)"""
    i, dim, hkv, heads, rows, ctx, window, use_sinks, causal, part, cache, block = case
    say("random case", case)
    fp8 = cache == torch.float8_e4m3fn
    batch = Batch(entries=tuple((n, rows) for n in ctx), tokens=len(ctx) * rows + 2,
                  reqs=len(ctx) + 1, heads=heads, kv_heads=hkv, head_dim=dim, block=block,
                  window=window, sinks=use_sinks, causal=causal)
    step = synthetic(batch, "cuda", torch.bfloat16, seed=100 + i, pool_pages=2048,
                     cache_dtype=cache if fp8 else None)
    if fp8:
        out = kvpath.paged_attention_fp8(*step.args, step.kv_scale, partition=part)
    else:
        out = kvpath.paged_attention(*step.args, partition=part)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    assert torch.equal(out[batch.n_rows:].cpu(), torch.zeros_like(out[batch.n_rows:].cpu()))
    atol, rtol = (FP8_ATOL, FP8_RTOL) if fp8 else (BF16_ATOL, BF16_RTOL)
    _check_against_oracle(out, step.args, None, atol, rtol, step.kv_scale, label=f"case {i}")


@pytest.mark.parametrize("dtype,dim,part", [
    (torch.float32, 64, 32),     # f32 partials, the general reduce (20+ partitions)
    (torch.float32, 64, 512),    # f32 partials, the few-partition reduce
    (torch.float16, 40, 32),     # f16: generic kernel, f32 partials
    (torch.bfloat16, 96, 32),    # bf16 q at a head dim the MFMA kernels do not take: the
    (torch.bfloat16, 96, 512),   # generic kernel with bf16 partials, both reduces
])
def test_generic_kernel_partials(dtype, dim, part) -> None:
    """The VALU kernel's partial formats through both reduce kernels: f32 partials for fp32 and
    f16 steps, bf16 partials for a bf16 q (any head dim), against the fp64 truth. Decode and
    verify rows, GQA 4, sinks, contexts up to ~700 keys."""
    say("generic partials", dtype, dim, part)
    batch = Batch(entries=((690, 1), (333, 4), (31, 1), (512, 3)), tokens=11, reqs=5, heads=8,
                  kv_heads=2, head_dim=dim, block=16, sinks=True)
    args = step_args(batch, "cuda", dtype, seed=dim + part)
    out = kvpath.paged_attention(*args, partition=part)
    torch.cuda.synchronize()
    truth = oracle.paged_attention(*step_args(batch, "cpu", torch.float64, seed=dim + part))
    got = out.double().cpu()
    assert torch.equal(out[batch.n_rows:].cpu(), torch.zeros_like(out[batch.n_rows:].cpu()))
    atol, rtol = {torch.float32: (2e-5, 1e-5), torch.float16: (1e-3, 1e-3),
                  torch.bfloat16: (BF16_ATOL, BF16_RTOL)}[dtype]
    err = (got - truth).abs()
    assert bool((err <= atol + rtol * truth.abs()).all()), (dtype, dim, part, err.max().item())


@pytest.mark.parametrize("part,heads,ctx", [
    (416, 16, (1289, 607, 1999)),   # 13 blocks per partition: three or four per wave
    (512, 4, (900, 1500, 33)),
    (0, 8, (2500, 1210, 857, 40)),
])
def test_decode_d256_multi_block_waves(part, heads, ctx) -> None:
    """bf16 decode at D 256 with partitions of several 32-key blocks per wave, so each wave
    refills its K registers inside the block loop (the path whose untracked K loads once had
    their destinations copied and reused before the wait: a GPU memory fault). Fused append,
    split-KV and reduce, against the fp64 oracle."""
    say("decode D256", part, heads, ctx)
    batch = Batch(entries=tuple((n, 1) for n in ctx), tokens=len(ctx) + 2, reqs=len(ctx) + 1,
                  heads=heads, kv_heads=2, head_dim=256, block=16, sinks=True)
    step = synthetic(batch, "cuda", torch.bfloat16, seed=400 + heads, pool_pages=1024)
    out = kvpath.paged_attention(*step.args, partition=part)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    assert torch.equal(out[batch.n_rows:].cpu(), torch.zeros_like(out[batch.n_rows:].cpu()))
    _check_against_oracle(out, step.args, None, BF16_ATOL, BF16_RTOL, None, label=f"D256 {part}")


def _many_entry_cases():
    """(label, dim, kv_heads, heads, rows, contexts, sinks, causal): multi-row bf16 steps of two
    to four row tiles per entry over many entries (contexts from one key), MQA, D 64 and 256,
    and the drafter's non-causal block."""
    g = torch.Generator().manual_seed(77)

    def ctx(n, lo, hi):
        return tuple(torch.randint(lo, hi + 1, (n,), generator=g).tolist())

    return [
        ("200 entries, short contexts", 128, 8, 32, 8, ctx(200, 1, 700), False, True),
        ("257 entries", 128, 8, 32, 5, ctx(257, 1, 900), True, True),
        ("16 entries, drafter", 128, 8, 32, 16, ctx(16, 100, 3000), False, False),
        ("MQA, G 8", 128, 1, 8, 6, ctx(24, 40, 2500), True, True),
        ("D 64", 64, 8, 64, 4, ctx(40, 1, 2000), True, True),
        ("D 256", 256, 2, 8, 12, ctx(12, 300, 1800), False, True),
    ]


@pytest.mark.parametrize("case", _many_entry_cases(), ids=lambda c: c[0])
def test_multi_row_many_entries(case) -> None:
    """Verify-shaped steps over many entries of uneven (down to one-key) contexts, with the
    library's partition choice: against the fp64 oracle, pad rows exactly zero."""
    label, dim, hkv, heads, rows, ctx, use_sinks, causal = case
    say("many entries", label)
    batch = Batch(entries=tuple((max(0, n - rows), rows) for n in ctx), tokens=len(ctx) * rows + 3,
                  reqs=len(ctx) + 1, heads=heads, kv_heads=hkv, head_dim=dim, block=16,
                  window=0, sinks=use_sinks, causal=causal)
    step = synthetic(batch, "cuda", torch.bfloat16, seed=300 + len(ctx), pool_pages=8192)
    out = kvpath.paged_attention(*step.args)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    assert torch.equal(out[batch.n_rows:].cpu(), torch.zeros_like(out[batch.n_rows:].cpu()))
    _check_against_oracle(out, step.args, None, BF16_ATOL, BF16_RTOL, None, label=label)


@pytest.mark.parametrize("block", [32, 64])
@pytest.mark.parametrize("rows,cache", [(1, torch.bfloat16), (16, torch.bfloat16), (1, torch.float8_e4m3fn),
                                        (5, torch.float8_e4m3fn)])
def test_larger_pages(block, rows, cache) -> None:
    """Pages of 32 and 64 tokens (kelpie's block size is per model): decode, verify and fp8 steps
    against the fp64 oracle, contexts ending mid-page."""
    say("block", block, rows, cache)
    fp8 = cache == torch.float8_e4m3fn
    ctx = (1, 31, 64, 100, 517, 1000)
    batch = Batch(entries=tuple((n, rows) for n in ctx), tokens=len(ctx) * rows + 2,
                  reqs=len(ctx) + 1, heads=32, kv_heads=8, head_dim=128, block=block, window=0,
                  sinks=True)
    step = synthetic(batch, "cuda", torch.bfloat16, seed=block + rows, pool_pages=512,
                     cache_dtype=cache if fp8 else None)
    if fp8:
        out = kvpath.paged_attention_fp8(*step.args, step.kv_scale)
    else:
        out = kvpath.paged_attention(*step.args)
    torch.cuda.synchronize()
    assert torch.equal(out[batch.n_rows:].cpu(), torch.zeros_like(out[batch.n_rows:].cpu()))
    atol, rtol = (FP8_ATOL, FP8_RTOL) if fp8 else (BF16_ATOL, BF16_RTOL)
    _check_against_oracle(out, step.args, None, atol, rtol, step.kv_scale, label=f"block {block}")


def test_graph_capture_replays_a_new_plan() -> None:
    """Capture the op once, write a different plan of the same shape into the captured buffers,
    replay several times with eager work in between; each replay equals the eager result."""
    say("graph capture")
    entries = [(40, 1), (130, 1), (7, 1), (300, 1), (1, 1), (16, 1), (17, 1), (600, 1)]
    first = Batch(entries=tuple(entries), tokens=8, reqs=8, heads=32, kv_heads=8, head_dim=128,
                  block=16, sinks=False)
    second = Batch(entries=tuple(entries[::-1]), tokens=8, reqs=8, heads=32, kv_heads=8,
                   head_dim=128, block=16, sinks=False)
    static = list(step_args(first, "cuda", torch.bfloat16, seed=10))
    fresh = step_args(second, "cuda", torch.bfloat16, seed=11)
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
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        eager = kvpath.paged_attention(*static)
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager)


def test_config5_copy_blocks_bit_exact() -> None:
    """Config 5's cache maintenance: 4096 seeded (src, dst) pairs over the 128k-context pool,
    src among live pages, dst among free pages; the whole member bit-exact vs the C oracle."""
    say("config 5 copy_blocks")
    batch, extra = config_batch(5)
    step = synthetic(batch, "cuda", torch.bfloat16, seed=5, pool_pages=extra["pool_pages"])
    src, dst = copy_pairs(step, extra["copy_pairs"])
    want = compact_member(step.kv_member)
    kvbytes.copy_blocks(want, src.cpu(), dst.cpu())
    kvpath.copy_blocks(step.kv_member, src, dst)
    torch.cuda.synchronize()
    got = compact_member(step.kv_member)
    assert torch.equal(got.contiguous().view(torch.uint8), want.contiguous().view(torch.uint8))


@pytest.mark.parametrize("rows,heads,dim,window,partition,causal", [
    (1, 32, 128, 0, 0, True),       # decode: the append runs inside the decode kernel
    (16, 32, 128, 0, 0, True),      # verify-shaped: inside the multi-row kernel, per partition
    (16, 32, 128, 0, 0, False),     # the drafter's non-causal block
    (16, 32, 128, 0, 1 << 16, True),  # ... one partition: direct output
    (16, 32, 256, 0, 0, True),      # verify-shaped at D 256
    (7, 64, 64, 40, 0, True),       # multi-row, D 64, window
    (16, 64, 64, 0, 0, True),       # gpt-oss 1 + 15 rows: two workgroups per partition
    (16, 64, 64, 128, 0, True),     # ... with its sliding window
    (16, 64, 64, 0, 0, False),      # ... the drafter's non-causal block
    (24, 64, 64, 0, 1 << 16, True),  # three workgroups, one partition: direct output
    (300, 32, 128, 0, 0, True),     # prefill-shaped: append launch, then two tiles per wave
    (300, 32, 128, 0, 1 << 16, True),  # ... one partition: direct output with the append
])
def test_fused_append_step(rows, heads, dim, window, partition, causal) -> None:
    """The whole op (append inside the decode kernel or the verify kernel, or launched before the
    prefill kernel): the pool rows at slot_mapping hold k, v bit-exact, nothing else in the pool
    changes, pad rows are exact zeros, and the output matches the fp64 oracle and the two-step
    path (write_kv, then attend)."""
    say("fused append", rows, heads, dim, window, partition, causal)
    base, _ = config_batch(2)
    entries = tuple((n, rows) for n, _ in base.entries[:6]) + ((0, rows), (15, min(rows, 3)))
    n_rows = sum(r for _, r in entries)
    batch = Batch(entries=entries, tokens=n_rows + 4, reqs=len(entries) + 2, heads=heads,
                  kv_heads=8, head_dim=dim, block=16, window=window, sinks=False, causal=causal)
    step = synthetic(batch, "cuda", torch.bfloat16, seed=21 + rows, pool_pages=8192)
    q, k, v, kv_member, rr, pos, qsl, lens, table, slots, window, sinks, causal = step.args
    before = compact_member(kv_member)
    fused = kvpath.paged_attention(*step.args, partition=partition)
    torch.cuda.synchronize()
    assert torch.equal(fused[batch.n_rows:].cpu(), torch.zeros_like(fused[batch.n_rows:].cpu()))
    want = before.clone()
    live = slots[: batch.n_rows].cpu()
    kvbytes.kv_append(want, k[: batch.n_rows].cpu(), v[: batch.n_rows].cpu(), live)
    got = compact_member(kv_member)
    assert torch.equal(got[1:].contiguous().view(torch.int16), want[1:].contiguous().view(torch.int16))
    two_step = kvpath.attend(q, kv_member, rr, qsl, lens, table, window, sinks, causal,
                             partition=partition)
    assert torch.equal(fused.cpu(), two_step.cpu())
    _check_against_oracle(fused, step.args, [0, 3, 5, 6, 7], BF16_ATOL, BF16_RTOL,
                          label="fused append")
