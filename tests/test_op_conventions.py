"""kvpath's torch ops against kelpie's op conventions (kernels/conventions.py:26-33): a fake for
meta tracing, samples that opcheck runs, and a backward that raises (ops/paged_attention.py:
376-385; the path is inference-only).

CPU: the fakes' shape rule under FakeTensorMode and the backward's refusal. GPU: torch.library.
opcheck (schema and mutation, fake against the real kernel, autograd registration, AOT dispatch
with dynamic shapes) on both ops at the reference's SAMPLE_BATCH and at a decode and a verify
sample, and `.backward()` through the op raising NotImplementedError.
"""

from __future__ import annotations

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import kvpath
from workloads import SAMPLE_BATCH, Batch, step_args, synthetic

DECODE = Batch(entries=((100, 1), (37, 1), (600, 1)), tokens=4, reqs=4, heads=32, kv_heads=8,
               head_dim=128, block=16, sinks=False)
VERIFY = Batch(entries=((300, 16), (45, 16)), tokens=32, reqs=2, heads=32, kv_heads=8,
               head_dim=128, block=16, sinks=False)


def _fake_args(args: tuple, mode: FakeTensorMode) -> tuple:
    return tuple(mode.from_tensor(a).to("cuda") if isinstance(a, torch.Tensor) else a
                 for a in args)


@pytest.mark.parametrize("batch", [SAMPLE_BATCH, DECODE, VERIFY])
def test_fake_shape_rule(batch) -> None:
    """Under FakeTensorMode (no kernel runs) both ops give [T, H * D] in q's dtype on q's device
    (ops/paged_attention.py:248-267)."""
    args = step_args(batch, "cpu", torch.bfloat16)
    mode = FakeTensorMode()
    with mode:
        fake = _fake_args(args, mode)
        out = torch.ops.kvpath.paged_attention(*fake)
        scale = torch.empty(fake[3].shape[0], 2, fake[3].shape[3], device="cuda")
        out8 = torch.ops.kvpath.paged_attention_fp8(*fake, scale)
    for o in (out, out8):
        assert tuple(o.shape) == (batch.tokens, batch.heads * batch.head_dim)
        assert o.dtype == torch.bfloat16 and o.device.type == "cuda"


def test_ops_are_registered_for_every_key_they_need() -> None:
    """The ops (registered in C++, libkvpath_torch.so: paged attention and write_kv, each plain
    and fp8) have a ROCm kernel, a CPU kernel that refuses, an Autograd kernel (the attention
    ops' backward raises, exercised on the GPU below) and a fake; the attention schema is
    kelpie's 13 arguments with kv_member (and kv_scale) the only ones written."""
    from torch._library.simple_registry import singleton

    for name in ("kvpath::paged_attention", "kvpath::paged_attention_fp8", "kvpath::write_kv",
                 "kvpath::write_kv_fp8"):
        for key in ("CUDA", "CPU", "Autograd"):
            assert torch._C._dispatch_has_kernel_for_dispatch_key(name, key), (name, key)
        assert singleton.find(name).fake_impl.kernel is not None, name
    schema = torch.ops.kvpath.paged_attention.default._schema
    assert [a.name for a in schema.arguments] == [
        "q", "k", "v", "kv_member", "row_request", "positions", "query_start_loc", "seq_lens",
        "block_table", "slot_mapping", "window", "sinks", "causal", "partition"]
    written = [a.name for a in schema.arguments if a.alias_info and a.alias_info.is_write]
    assert written == ["kv_member"]
    schema8 = torch.ops.kvpath.paged_attention_fp8.default._schema
    assert [a.name for a in schema8.arguments if a.alias_info and a.alias_info.is_write] == [
        "kv_member", "kv_scale"]


def _samples(fp8: bool) -> list[tuple]:
    out = []
    if not fp8:  # the fp8 kernels need D of 64, 128 or 256; SAMPLE_BATCH has D 32
        out.append((step_args(SAMPLE_BATCH, "cuda", torch.bfloat16), None))
    for i, batch in enumerate((DECODE, VERIFY)):
        step = synthetic(batch, "cuda", torch.bfloat16, seed=70 + i, pool_pages=128,
                         cache_dtype=torch.float8_e4m3fn if fp8 else None)
        out.append((step.args, step.kv_scale))
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("fp8", [False, True])
def test_opcheck(fp8) -> None:
    """torch.library.opcheck on the op: schema (kv_member, and kv_scale for fp8, are the only
    arguments written), fake against the real kernel, autograd registration, AOT dispatch with
    dynamic shapes."""
    op = torch.ops.kvpath.paged_attention_fp8.default if fp8 else \
        torch.ops.kvpath.paged_attention.default
    # opcheck's schema test detects mutation with arithmetic torch has no float8 kernels for; the
    # fp8 op's mutations are checked byte for byte instead (only kv_member and kv_scale change).
    utils = ("test_faketensor", "test_autograd_registration", "test_aot_dispatch_dynamic") \
        if fp8 else ("test_schema", "test_faketensor", "test_autograd_registration",
                     "test_aot_dispatch_dynamic")
    for args, scale in _samples(fp8):
        full = args + (scale,) if fp8 else args
        torch.library.opcheck(op, full, test_utils=utils)
        if fp8:
            before = [a.clone() if isinstance(a, torch.Tensor) else a for a in full]
            op(*full)
            torch.cuda.synchronize()
            for i, (a, b) in enumerate(zip(full, before)):
                if not isinstance(a, torch.Tensor) or i in (3, 13):  # kv_member, kv_scale
                    continue
                assert torch.equal(a.view(torch.uint8) if a.dtype == torch.float8_e4m3fn else a,
                                   b.view(torch.uint8) if b.dtype == torch.float8_e4m3fn else b), i


@pytest.mark.gpu
@pytest.mark.parametrize("fp8", [False, True])
def test_backward_through_the_op_raises(fp8) -> None:
    """q requiring grad: the forward runs (and bumps kv_member's version, an in-place write), the
    output requires grad, and `.backward()` raises NotImplementedError naming the op."""
    step = synthetic(DECODE, "cuda", torch.bfloat16, seed=77, pool_pages=128,
                     cache_dtype=torch.float8_e4m3fn if fp8 else None)
    args = step.args
    q = args[0].detach().requires_grad_(True)
    version = args[3]._version
    out = (kvpath.paged_attention_fp8(q, *args[1:], step.kv_scale) if fp8 else
           kvpath.paged_attention(q, *args[1:]))
    assert out.requires_grad and args[3]._version > version
    with pytest.raises(NotImplementedError, match="no backward"):
        out.float().sum().backward()
