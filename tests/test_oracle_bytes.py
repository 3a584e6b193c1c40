"""The C byte oracle, pinned (oracle/kvbytes.c).

e4m3 against torch's float8_e4m3fn cast on every bf16 bit pattern and the format's boundary
values; append / gather / copy_blocks against torch's own index_copy_ / index_select / indexing
(the library routines the reference uses, ops/paged_attention.py:44-54, 172-177) and a
token-valued pool read back through the block tables (the check_core_loop.py:205-229 pattern);
fp8 quantize-on-append against closed forms computed with torch ops, order independence, scale
monotonicity and the rounding-error bound.
"""

from __future__ import annotations

import pytest
import torch

from workloads import Batch, step_args
from oracle import attention as oracle_attn
from oracle import kvbytes


def _arena(pages: int, block: int, heads: int, dim: int, dtype, members: int = 2) -> torch.Tensor:
    """A member view laid out as the engine's arena: [pages, block, members, 2, Hkv, D], member 1."""
    arena = torch.zeros(pages, block, members, 2, heads, dim, dtype=dtype)
    return arena[:, :, members - 1].permute(0, 2, 1, 3, 4)


# ---- e4m3 ----------------------------------------------------------------------------------------


def test_e4m3_every_bf16_pattern_matches_torch() -> None:
    bits = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16)
    x = bits.view(torch.bfloat16).float()
    x = x[torch.isfinite(x)].clamp(-448, 448)
    got = kvbytes.e4m3_encode(x)
    want = x.to(torch.float8_e4m3fn).view(torch.uint8)
    assert torch.equal(got, want)


def test_e4m3_boundaries_match_torch() -> None:
    vals = [0.0, -0.0, 448.0, -448.0, 447.9, 416.0, 432.0, 2.0 ** -6, 2.0 ** -7, 2.0 ** -9,
            2.0 ** -10, 1.5 * 2.0 ** -10, 2.0 ** -10 * 1.0001, 3 * 2.0 ** -10, 1.0625, 1.1875,
            -1.0625, 0.96875, 240.0, 256.0, 272.0, 288.0, 1e-30]
    x = torch.tensor(vals, dtype=torch.float32)
    assert torch.equal(kvbytes.e4m3_encode(x), x.to(torch.float8_e4m3fn).view(torch.uint8))


def test_e4m3_random_f32_and_decode() -> None:
    g = torch.Generator().manual_seed(0)
    x = (torch.randn(1_000_000, generator=g) * torch.exp(torch.randn(1_000_000, generator=g) * 3))
    x = x.clamp(-448, 448)
    assert torch.equal(kvbytes.e4m3_encode(x), x.to(torch.float8_e4m3fn).view(torch.uint8))
    every = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    got = kvbytes.e4m3_decode(every)
    want = every.view(torch.float8_e4m3fn).float()
    nan = torch.isnan(want)
    assert torch.equal(torch.isnan(got), nan)
    assert torch.equal(got[~nan], want[~nan])


def test_fp8_quantize_is_the_clamped_scaled_cast() -> None:
    """One value against a page scale through its reciprocal: x * r in f32, clamped to +-448,
    then torch's e4m3 cast; 0 when the reciprocal is 0 (an all-zero page). Values reach past
    the clamp on both sides, and a reciprocal that is not a power of two rounds the product."""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(4000, generator=g) * torch.exp(torch.randn(4000, generator=g) * 2)
    for r in (0.0, 1.0, 3.0, 448.0 / 3.7, 2.0 ** -9, 1.0 / 0.0175):
        rr = torch.tensor(r, dtype=torch.float32)
        want = (x * rr).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8)
        if r == 0.0:
            want = torch.zeros_like(want)
        got = torch.tensor([kvbytes.fp8_quantize(v, float(rr)) for v in x.tolist()], dtype=torch.uint8)
        assert torch.equal(got, want), r


# ---- append / gather / copy_blocks ----------------------------------------------------------------


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_append_matches_index_copy(dtype) -> None:
    """Bytes written by the oracle == torch index_copy_ on both members (write_kv, ops:44-54)."""
    g = torch.Generator().manual_seed(1)
    pages, block, heads, dim = 9, 4, 3, 16
    a = _arena(pages, block, heads, dim, dtype)
    b = _arena(pages, block, heads, dim, dtype)
    fill = torch.randn(a.shape, generator=g).to(dtype)
    a.copy_(fill)
    b.copy_(fill)
    slots = torch.tensor([5, 17, 3, 35, 3, 20], dtype=torch.int32)  # 3 twice: two pad rows
    k = torch.randn(6, heads, dim, generator=g).to(dtype)
    v = torch.randn(6, heads, dim, generator=g).to(dtype)
    k[4], v[4] = k[2], v[2]  # the two pad rows carry the same values, so order cannot matter
    kvbytes.kv_append(a, k, v, slots)
    oracle_attn.write_kv(b, k, v, slots)
    assert torch.equal(a.contiguous().view(torch.uint8), b.contiguous().view(torch.uint8))


def test_token_valued_pool_reads_back_through_tables() -> None:
    """Every row writes its token id at its slot; reading positions 0..p of each entry through
    its block table returns exactly the ids written (the check_core_loop.py:205-229 oracle)."""
    batch = Batch(entries=((13, 3), (0, 5), (30, 1)), tokens=10, reqs=4, heads=2, kv_heads=1,
                  head_dim=4, block=4)
    args = step_args(batch, "cpu", torch.float32, seed=7)
    kv_member, slots, table, qsl = args[3], args[9], args[8], args[6]
    seq_lens = args[7]
    # context rows get ids 1000*r + position, this step's rows the same rule
    flat_k, flat_v = oracle_attn.kv_views(kv_member)
    for r, (ctx, _) in enumerate(batch.entries):
        for p in range(ctx):
            s = int(table[r, p // 4]) * 4 + p % 4
            flat_k[s] = 1000 * r + p
            flat_v[s] = -(1000 * r + p)
    k = torch.zeros(10, 1, 4)
    v = torch.zeros(10, 1, 4)
    for r in range(3):
        for t in range(int(qsl[r]), int(qsl[r + 1])):
            pos = int(seq_lens[r]) - (int(qsl[r + 1]) - int(qsl[r])) + (t - int(qsl[r]))
            k[t], v[t] = 1000 * r + pos, -(1000 * r + pos)
    kvbytes.kv_append(kv_member, k, v, slots)
    width = table.shape[1]
    gk, gv = kvbytes.kv_gather(kv_member, table, width)
    for r, (ctx, rows) in enumerate(batch.entries):
        n = ctx + rows
        ids = torch.arange(n, dtype=torch.float32) + 1000 * r
        assert torch.equal(gk[r, :n, 0, 0], ids)
        assert torch.equal(gv[r, :n, 0, 0], -ids)


def test_gather_matches_index_select() -> None:
    """out[r, j] = K[table[r, j//block]*block + j%block] (ops:174-177 with index_select)."""
    batch = Batch(entries=((21, 2), (6, 1)), tokens=4, reqs=3, heads=4, kv_heads=2, head_dim=8,
                  block=4)
    args = step_args(batch, "cpu", torch.bfloat16, seed=2)
    kv_member, table = args[3], args[8]
    width = table.shape[1]
    gk, gv = kvbytes.kv_gather(kv_member, table, width)
    flat_k, flat_v = oracle_attn.kv_views(kv_member)
    slots = (table.long()[:, :, None] * 4 + torch.arange(4)).reshape(-1)
    assert torch.equal(gk.view(torch.int16).reshape(-1, 2, 8),
                       flat_k.index_select(0, slots).view(torch.int16))
    assert torch.equal(gv.view(torch.int16).reshape(-1, 2, 8),
                       flat_v.index_select(0, slots).view(torch.int16))


def test_copy_blocks_closed_form() -> None:
    g = torch.Generator().manual_seed(3)
    kv = _arena(12, 4, 2, 8, torch.bfloat16)
    kv.copy_(torch.randn(kv.shape, generator=g).to(torch.bfloat16))
    scale = torch.rand(12, 2, 2, generator=g)
    before, sbefore = kv.clone(), scale.clone()
    src = torch.tensor([1, 4, 7], dtype=torch.int32)
    dst = torch.tensor([9, 2, 11], dtype=torch.int32)
    kvbytes.copy_blocks(kv, src, dst, scale)
    want, swant = before.clone(), sbefore.clone()
    want[dst.long()] = before[src.long()]
    swant[dst.long()] = sbefore[src.long()]
    assert torch.equal(kv.view(torch.int16), want.view(torch.int16))
    assert torch.equal(scale, swant)


# ---- fp8 quantize-on-append ----------------------------------------------------------------------


def _fp8_member(pages=6, block=16, heads=2, dim=16):
    arena = torch.zeros(pages, block, 2, 2, heads, dim, dtype=torch.uint8)
    member = arena.view(torch.float8_e4m3fn)[:, :, 1].permute(0, 2, 1, 3, 4)
    return member, torch.zeros(pages, 2, heads, dtype=torch.float32)


def _bf16(*shape, g, outliers=0.0):
    x = torch.randn(*shape, generator=g)
    if outliers:
        x = torch.where(torch.rand(*shape, generator=g) < outliers, x * 20, x)
    return x.to(torch.bfloat16)


def test_fp8_fresh_page_closed_form() -> None:
    """A step writing rows 0..3 of a page: scale = absmax/448 per (member, head), bytes = torch's
    e4m3 cast of clamp(x * (1 / scale))."""
    g = torch.Generator().manual_seed(4)
    kv, scale = _fp8_member()
    k, v = _bf16(4, 2, 16, g=g), _bf16(4, 2, 16, g=g)
    slots = torch.arange(2 * 16, 2 * 16 + 4, dtype=torch.int32)  # page 2 rows 0..3
    kvbytes.kv_append_fp8(kv, scale, k, v, slots)
    for m, x in enumerate((k, v)):
        for h in range(2):
            xf = x[:, h].float()
            s = xf.abs().max() / 448.0
            assert scale[2, m, h] == s
            want = (xf * (1.0 / s)).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8)
            assert torch.equal(kv[2, m, :4, h].view(torch.uint8), want)


def _growth(s_old: torch.Tensor, t: torch.Tensor) -> int:
    """The smallest k >= 1 with s_old * 2^k >= t, by exact power-of-two products."""
    k = 1
    while bool(torch.ldexp(s_old, torch.tensor(k)) < t):
        k += 1
    return k


def test_fp8_requantizes_on_scale_growth() -> None:
    """Rows 0..3, then row 4 with a larger absmax: the scale grows by the smallest power of two
    2^k that covers absmax/448, rows 0..3 become e4m3(clamp(f32(q) * 2^-k)) and row 4
    e4m3(clamp(x * (1 / s_new))); a later smaller row keeps the scale."""
    g = torch.Generator().manual_seed(5)
    kv, scale = _fp8_member()
    k1, v1 = _bf16(4, 2, 16, g=g), _bf16(4, 2, 16, g=g)
    kvbytes.kv_append_fp8(kv, scale, k1, v1, torch.arange(16, 20, dtype=torch.int32))
    old_bytes, old_scale = kv[1].clone(), scale[1].clone()
    k2, v2 = (_bf16(1, 2, 16, g=g).float() * 8).to(torch.bfloat16), _bf16(1, 2, 16, g=g)
    kvbytes.kv_append_fp8(kv, scale, k2, v2, torch.tensor([20], dtype=torch.int32))
    grew = 0
    for m, x in enumerate((k2, v2)):
        for h in range(2):
            s_old = old_scale[m, h]
            t = x[0, h].float().abs().max() / 448.0
            k = _growth(s_old, t) if t > s_old else 0
            s_new = torch.ldexp(s_old, torch.tensor(k))
            assert scale[1, m, h] == s_new
            old = old_bytes[m, :4, h].float()
            if k:
                grew += 1
                want = torch.ldexp(old, torch.tensor(-k)).clamp(-448, 448).to(torch.float8_e4m3fn)
            else:
                want = old_bytes[m, :4, h]
            assert torch.equal(kv[1, m, :4, h].view(torch.uint8), want.view(torch.uint8))
            new = (x[0, h].float() * (1.0 / s_new)).clamp(-448, 448).to(torch.float8_e4m3fn)
            assert torch.equal(kv[1, m, 4, h].view(torch.uint8), new.view(torch.uint8))
    assert grew >= 2 and bool((scale[1, 0] > old_scale[0]).all())  # K grew (x8); the rule fired


def test_fp8_growth_keeps_dequantized_values() -> None:
    """A scale growth is an exponent shift: every requantized element whose value stays an e4m3
    normal dequantizes to exactly what it did before (no rounding compounds over a decode
    stream); a fresh page's largest element maps to 448 and comes back to within the f32
    rounding of its scale."""
    g = torch.Generator().manual_seed(9)
    kv, scale = _fp8_member(pages=3)
    before_vals = None
    for row in range(16):
        k = (_bf16(1, 2, 16, g=g).float() * (1.0 + row / 3)).to(torch.bfloat16)
        v = _bf16(1, 2, 16, g=g)
        if row == 0:
            kvbytes.kv_append_fp8(kv, scale, k, v, torch.tensor([16], dtype=torch.int32))
            first = k[0].float().abs().amax(dim=-1)
            deq0 = kvbytes.e4m3_decode(kv[1, 0, 0].contiguous()).reshape(2, 16) * scale[1, 0][:, None]
            torch.testing.assert_close(deq0.abs().amax(dim=-1), first, rtol=2.0 ** -23, atol=0)
        else:
            kvbytes.kv_append_fp8(kv, scale, k, v, torch.tensor([16 + row], dtype=torch.int32))
        q = kv[1, 0, :row].contiguous()
        vals = kvbytes.e4m3_decode(q).reshape(row, 2, 16) * scale[1, 0][None, :, None]
        if before_vals is not None and row > 1:
            prev = before_vals[:row - 1]
            now = vals[:row - 1]
            # elements that are e4m3 normals after the shift (|q| >= 2^-6) keep their value
            normal = kvbytes.e4m3_decode(q[:row - 1]).reshape(row - 1, 2, 16).abs() >= 2.0 ** -6
            assert torch.equal(now[normal], prev[normal]), row
        before_vals = kvbytes.e4m3_decode(kv[1, 0, :row + 1].contiguous()).reshape(row + 1, 2, 16) \
            * scale[1, 0][None, :, None]
    assert bool((scale[1, 0] > 0).all())


def test_fp8_step_order_independent_and_monotone() -> None:
    """Permuting a step's rows gives the same bytes and scales; scales never shrink."""
    g = torch.Generator().manual_seed(6)
    kv_a, sc_a = _fp8_member(pages=8)
    kv_b, sc_b = _fp8_member(pages=8)
    history = []
    for step in range(5):
        n = 6
        # three pages, two rows each, rows 2*step, 2*step+1 of pages 1, 3, 5
        slots = torch.tensor([p * 16 + 2 * step + i for p in (1, 3, 5) for i in range(2)],
                             dtype=torch.int32)
        k, v = _bf16(n, 2, 16, g=g, outliers=0.05), _bf16(n, 2, 16, g=g, outliers=0.05)
        kvbytes.kv_append_fp8(kv_a, sc_a, k, v, slots)
        perm = torch.randperm(n, generator=g)
        kvbytes.kv_append_fp8(kv_b, sc_b, k[perm], v[perm], slots[perm])
        history.append(sc_a.clone())
    assert torch.equal(kv_a.view(torch.uint8), kv_b.view(torch.uint8))
    assert torch.equal(sc_a, sc_b)
    for before, after in zip(history, history[1:]):
        assert bool((after >= before).all())


def test_fp8_error_bound_first_write() -> None:
    """|dequant - x| <= half an e4m3 step: 2^-4 |x| for normals, s * 2^-10 below 2^-6 * s."""
    g = torch.Generator().manual_seed(7)
    kv, scale = _fp8_member(pages=3)
    k, v = _bf16(16, 2, 16, g=g, outliers=0.01), _bf16(16, 2, 16, g=g, outliers=0.01)
    kvbytes.kv_append_fp8(kv, scale, k, v, torch.arange(16, 32, dtype=torch.int32))
    for m, x in enumerate((k, v)):
        deq = kvbytes.e4m3_decode(kv[1, m].contiguous()).reshape(16, 2, 16) * scale[1, m].reshape(1, 2, 1)
        err = (deq - x.float()).abs()
        bound = torch.maximum(x.float().abs() * 2 ** -4, scale[1, m].reshape(1, 2, 1) * 2 ** -10)
        assert bool((err <= bound * (1 + 1e-6)).all())


def test_fp8_fresh_page_discards_stale_scale() -> None:
    g = torch.Generator().manual_seed(8)
    kv, scale = _fp8_member(pages=3)
    scale.fill_(1000.0)  # a previous owner's scale
    k, v = _bf16(1, 2, 16, g=g), _bf16(1, 2, 16, g=g)
    kvbytes.kv_append_fp8(kv, scale, k, v, torch.tensor([32], dtype=torch.int32))  # page 2 row 0
    assert torch.equal(scale[2, 0], k[0].float().abs().amax(dim=-1) / 448.0)
    assert bool((scale[1] == 1000.0).all())  # untouched pages keep theirs
