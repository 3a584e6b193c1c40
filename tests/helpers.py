"""Shared test helpers: golden-case batches and inputs, digests, the grading rule."""

from __future__ import annotations

import hashlib

import torch

from kvpath.paged_attention import KV_MEMBERS
from workloads import GARBAGE, Batch

PLAN = ("row_request", "positions", "query_start_loc", "seq_lens", "block_table", "slot_mapping")


def batch_of(meta_batch: dict) -> Batch:
    kw = dict(meta_batch)
    kw["entries"] = tuple(tuple(e) for e in kw["entries"])
    return Batch(**kw)


def golden_batch(name: str, meta: dict) -> Batch:
    return batch_of(meta[name]["batch"])


def golden_args(name: str, golden: tuple[dict, dict], device: str | torch.device,
                dtype: torch.dtype) -> tuple:
    """The op's 13 arguments for golden case `name`, rebuilt from the fixture's bf16 draw: the
    arena [pages, block, 2 members, K/V, Hkv, D] is GARBAGE with this layer (member 1) holding
    the stored values, so the kv_member is a strided view as the reference's sample() lays it
    out; fp32 and fp64 cases are exact upcasts of the bf16 values (sinks stay f32)."""
    meta, arrays = golden
    b = golden_batch(name, meta)

    def stored(key: str) -> torch.Tensor:
        return torch.from_numpy(arrays[f"{name}/in_{key}"].copy())

    member = stored("member").view(torch.bfloat16).to(dtype)
    arena = torch.full((member.shape[0], b.block, 2, KV_MEMBERS, b.kv_heads, b.head_dim), GARBAGE,
                       dtype=dtype, device=device)
    kv_member = arena[:, :, 1].permute(0, 2, 1, 3, 4)
    kv_member.copy_(member.to(device))
    q, k, v = (stored(x).view(torch.bfloat16).to(device=device, dtype=dtype) for x in "qkv")
    plan = [stored(key).to(device) for key in PLAN]
    return (q, k, v, kv_member, *plan, b.window, stored("sinks").to(device), b.causal)


def digest(t: torch.Tensor) -> str:
    """sha256 of a CPU tensor's bytes; a strided (5-d member) view digests its whole storage."""
    if t.dim() == 5:  # digest the whole storage, read on the tensor's own device
        words = torch.empty(0, dtype=torch.uint8, device=t.device).set_(t.untyped_storage())
        data = words.cpu().numpy().tobytes()
    else:
        t = t.cpu()
        data = t.contiguous().view(torch.uint8).numpy().tobytes() if t.numel() else b""
    return hashlib.sha256(data).hexdigest()


def within(out: torch.Tensor, truth: torch.Tensor, atol: float, rtol: float) -> tuple[bool, float]:
    """|out - truth| <= atol + rtol * |truth| everywhere; returns (ok, worst excess ratio)."""
    o, t = out.double().cpu(), truth.double().cpu()
    err = (o - t).abs()
    bound = atol + rtol * t.abs()
    ratio = (err / bound).max().item() if err.numel() else 0.0
    return bool(torch.isfinite(o).all()) and ratio <= 1.0, ratio
