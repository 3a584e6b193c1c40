"""Shared test helpers: golden-case batches, digests, the grading rule."""

from __future__ import annotations

import hashlib

import torch

from reference_sample import SAMPLE_BATCH
from workloads import Batch


def batch_of(meta_batch: dict) -> Batch:
    kw = dict(meta_batch)
    kw["entries"] = tuple(tuple(e) for e in kw["entries"])
    return Batch(**kw)


def golden_batch(name: str, meta: dict) -> Batch:
    return SAMPLE_BATCH if name == "sample_batch" else batch_of(meta[name]["batch"])


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
