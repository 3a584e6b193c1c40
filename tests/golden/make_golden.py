"""Writes tests/golden/reference_cases.{npz,json}: input digests and outputs of the reference's
own `kelpie::paged_attention` body on the reference's own seeded `sample()`.

Run in the build container only (it imports the reference from /root/reference, which no GPU
box has):

    python tests/golden/make_golden.py

What it pins, that nothing else can: (1) that tests/reference_sample.py:sample reproduces the reference's
sample() draw for draw (sha256 of every input tensor's bytes, per dtype), and (2) the reference's
exact outputs -- fp64 (the truth), fp32 and bf16 -- and the bf16 pool after its write_kv, which
the CPU oracle (oracle/attention.py) must reproduce. Reference: kelpie/kelpie-models/
kelpie_models/kernels/ops/paged_attention.py:67-140 (op body), :270-373 (Batch, sample).
"""

from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np
import torch

REFERENCE = Path("/root/reference/kelpie/kelpie-models")
OUT = Path(__file__).resolve().parent

# (name, Batch kwargs, seed). Small shapes: the fixture holds every output value.
GPT_OSS = dict(heads=16, kv_heads=4, head_dim=64, block=16)  # gpt-oss-like, GQA 4, D 64
LLAMA = dict(heads=32, kv_heads=8, head_dim=128, block=16, sinks=False)
CASES = [
    ("sample_batch", None, 0),
    ("c1_tiny_decode", dict(entries=((16, 1), (63, 1), (128, 1), (254, 1)), tokens=4, reqs=4,
                            **LLAMA), 0),
    ("decode_padded", dict(entries=((37, 1), (90, 1), (1, 1), (16, 1), (64, 1)), tokens=8,
                           reqs=8, **GPT_OSS), 1),
    ("decode_window", dict(entries=((200, 1), (129, 1), (5, 1)), tokens=4, reqs=4, window=128,
                           **GPT_OSS), 2),
    ("verify_ragged", dict(entries=((40, 16), (30, 3), (7, 1), (50, 9)), tokens=32, reqs=4,
                           **GPT_OSS), 3),
    ("drafter", dict(entries=((40, 16), (30, 3), (7, 1), (50, 9)), tokens=32, reqs=4,
                     causal=False, **{**GPT_OSS, "sinks": False}), 4),
    ("prefill_mixed", dict(entries=((0, 20), (33, 1), (17, 5)), tokens=32, reqs=4, **GPT_OSS), 5),
    ("llama_verify", dict(entries=((100, 8),), tokens=8, reqs=1, **LLAMA), 6),
]


# Cases whose fp32 reference output is kept (fp32 is their config dtype); the others keep the
# fp64 truth (stored as fp32) and the bf16 output.
FP32_OUTPUTS = ("sample_batch", "c1_tiny_decode")


def digest(t: torch.Tensor) -> str:
    """sha256 of a tensor's bytes; a strided view digests its whole storage."""
    if t.dim() == 5:
        data = bytes(t.untyped_storage())
    else:
        data = t.contiguous().view(torch.uint8).numpy().tobytes() if t.numel() else b""
    return hashlib.sha256(data).hexdigest()


def main() -> int:
    sys.path.insert(0, str(REFERENCE))
    import kelpie_models.kernels.ops  # noqa: F401  (registers the op)

    pa = sys.modules["kelpie_models.kernels.ops.paged_attention"]
    reference = pa.paged_attention.reference
    arrays: dict[str, np.ndarray] = {}
    meta: dict[str, dict] = {}
    for name, kw, seed in CASES:
        batch = pa.SAMPLE_BATCH if kw is None else pa.Batch(**kw)
        entry = {"batch": {k: getattr(batch, k) for k in (
            "entries", "tokens", "reqs", "heads", "kv_heads", "head_dim", "block", "window",
            "sinks", "causal", "spare_pages")}, "seed": seed, "inputs": {}}
        for dtype in (torch.float64, torch.float32, torch.bfloat16):
            args = pa.sample(batch, "cpu", dtype, seed=seed)
            tag = str(dtype).removeprefix("torch.")
            entry["inputs"][tag] = [digest(a) if isinstance(a, torch.Tensor) else a
                                    for a in args]
            out = reference(*args)
            if dtype == torch.bfloat16:
                arrays[f"{name}/out_{tag}"] = out.view(torch.int16).numpy()
            elif dtype == torch.float64 or name in FP32_OUTPUTS:
                arrays[f"{name}/out_{tag}"] = out.to(torch.float32).numpy()
            if dtype == torch.bfloat16:
                entry["pool_after_bf16"] = digest(args[3])
        meta[name] = entry
        print(f"{name}: out {tuple(arrays[f'{name}/out_float64'].shape)}", flush=True)
    np.savez_compressed(OUT / "reference_cases.npz", **arrays)
    (OUT / "reference_cases.json").write_text(json.dumps(meta, indent=1) + "\n")
    print(f"wrote {OUT / 'reference_cases.npz'} and reference_cases.json")
    return 0


if __name__ == "__main__":
    sys.exit(main())
