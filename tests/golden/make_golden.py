"""Writes tests/golden/reference_cases.{npz,json} and tests/golden/reference_shapes.json from the
reference's own code: the inputs its seeded `sample()` draws, the outputs of its
`kelpie::paged_attention` body on them, and the shape tables of its per-op proof.

Run in the build container only (it imports the reference from /root/reference, which no GPU
box has):

    python tests/golden/make_golden.py

reference_cases.npz holds, per case, the bf16 draw as data: the layer's KV member
(`{case}/in_member`, int16 bit patterns, [pages, 2, block, Hkv, D]; the arena's other member is
GARBAGE everywhere), q/k/v (int16 bit patterns), the six int32 plan tensors and the f32 sinks.
The reference draws every value in fp32 and rounds it to bf16 before casting to the case dtype,
so its fp32 and fp64 samples are exact upcasts of the bf16 one; this script asserts that, and
the json keeps the sha256 of every input tensor per dtype so the tests can check the rebuilt
arguments against the reference's own. Outputs: the fp64 truth (`out_float64`, float64), the
fp32 output where fp32 is the case's dtype, the bf16 output (int16 bit patterns) and the digest
of the bf16 pool after its write_kv.

reference_shapes.json holds the per-op proof's case list (kelpie/scripts/bench_attention.py:
62-91, `shapes(random.Random(0))`, each at windows 0 and 128 plus the drafter's call) and its
timing buckets (`shapes(random.Random(1))` without the chunked, mixed and padded shapes,
:211-237), as the reference's own functions return them.

Reference: kelpie/kelpie-models/kelpie_models/kernels/ops/paged_attention.py:67-140 (op body),
:270-373 (Batch, sample, SAMPLE_BATCH).
"""

from __future__ import annotations

import hashlib
import importlib.util
import json
import random
import sys
from pathlib import Path

import numpy as np
import torch

REFERENCE = Path("/root/reference/kelpie")
OUT = Path(__file__).resolve().parent

# (name, Batch kwargs, seed). Small shapes: the fixture holds every input and output value.
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

# Cases whose fp32 reference output is kept (fp32 is their config dtype).
FP32_OUTPUTS = ("sample_batch", "c1_tiny_decode")
PLAN = ("row_request", "positions", "query_start_loc", "seq_lens", "block_table", "slot_mapping")


def digest(t: torch.Tensor) -> str:
    """sha256 of a tensor's bytes; a strided (5-d member) view digests its whole storage."""
    if t.dim() == 5:
        data = bytes(t.untyped_storage())
    else:
        data = t.contiguous().view(torch.uint8).numpy().tobytes() if t.numel() else b""
    return hashlib.sha256(data).hexdigest()


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().copy()


def store_inputs(name: str, args: tuple, wide: dict[str, tuple], arrays: dict) -> None:
    """The bf16 draw as arrays; asserts the fp32/fp64 draws are its exact upcasts and that the
    arena outside the member is GARBAGE (so the member alone rebuilds it)."""
    q, k, v, member = args[:4]
    for tag, other in wide.items():
        for a, b in zip(args, other):
            if isinstance(a, torch.Tensor) and a.is_floating_point() and a.dtype == torch.bfloat16:
                assert torch.equal(a.to(b.dtype), b), (name, tag)
            elif isinstance(a, torch.Tensor) and a.dim() != 5:
                assert torch.equal(a, b), (name, tag)
        arena = torch.empty(0, dtype=other[3].dtype).set_(other[3].untyped_storage())
        assert torch.equal(arena.view(member.shape[0], member.shape[2], 2, 2, member.shape[3],
                                      member.shape[4])[:, :, 1].permute(0, 2, 1, 3, 4),
                           member.to(other[3].dtype)), (name, tag)
    arena = torch.empty(0, dtype=torch.bfloat16).set_(member.untyped_storage())
    arena = arena.view(member.shape[0], member.shape[2], 2, 2, member.shape[3], member.shape[4])
    assert bool((arena[:, :, 0] == 64.0).all()), name  # the other member: GARBAGE throughout
    arrays[f"{name}/in_member"] = bits(member)
    arrays[f"{name}/in_q"] = bits(q)
    arrays[f"{name}/in_k"] = bits(k)
    arrays[f"{name}/in_v"] = bits(v)
    for key, t in zip(PLAN, args[4:10]):
        assert t.dtype == torch.int32, (name, key)
        arrays[f"{name}/in_{key}"] = t.numpy().copy()
    arrays[f"{name}/in_sinks"] = args[11].to(torch.float32).numpy().copy()


def reference_shapes(bench) -> dict:
    def rows(pairs):
        return [[label, {**kw, "entries": [list(e) for e in kw["entries"]]}] for label, kw in pairs]

    cases = [[label, {f: getattr(b, f) for f in ("entries", "tokens", "reqs", "heads", "kv_heads",
                                                 "head_dim", "block", "window", "sinks", "causal",
                                                 "spare_pages")}]
             for label, b in bench.cases()]
    for _, kw in cases:
        kw["entries"] = [list(e) for e in kw["entries"]]
    buckets = [[label, kw] for label, kw in rows(bench.shapes(random.Random(1)))
               if not ("chunk" in label or "mixed" in label or "(5 real)" in label)]
    return {"source": "kelpie/scripts/bench_attention.py: cases() (shapes(random.Random(0)), "
                      "windows 0 and 128, drafter at decode_extra) and the timing buckets "
                      "(shapes(random.Random(1)) without chunk/mixed/padded)",
            "attention": bench.GPT_OSS, "cases": cases, "buckets": buckets}


def main() -> int:
    sys.path.insert(0, str(REFERENCE / "kelpie-models"))
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
        drawn = {}
        for dtype in (torch.float64, torch.float32, torch.bfloat16):
            tag = str(dtype).removeprefix("torch.")
            drawn[tag] = pa.sample(batch, "cpu", dtype, seed=seed)
            entry["inputs"][tag] = [digest(a) if isinstance(a, torch.Tensor) else a
                                    for a in drawn[tag]]
        store_inputs(name, drawn["bfloat16"], {t: drawn[t] for t in ("float32", "float64")},
                     arrays)
        for tag, args in drawn.items():
            out = reference(*args)
            if tag == "bfloat16":
                arrays[f"{name}/out_{tag}"] = bits(out)
                entry["pool_after_bf16"] = digest(args[3])
            elif tag == "float64":
                arrays[f"{name}/out_{tag}"] = out.numpy().copy()
            elif name in FP32_OUTPUTS:
                arrays[f"{name}/out_{tag}"] = out.numpy().copy()
        meta[name] = entry
        print(f"{name}: member {arrays[f'{name}/in_member'].shape}, "
              f"out {arrays[f'{name}/out_float64'].shape}", flush=True)
    np.savez_compressed(OUT / "reference_cases.npz", **arrays)
    (OUT / "reference_cases.json").write_text(json.dumps(meta, indent=1) + "\n")

    spec = importlib.util.spec_from_file_location("bench_attention",
                                                  REFERENCE / "scripts" / "bench_attention.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    shapes = reference_shapes(bench)
    (OUT / "reference_shapes.json").write_text(json.dumps(shapes, indent=1) + "\n")
    print(f"wrote reference_cases.npz, reference_cases.json and reference_shapes.json "
          f"({len(shapes['cases'])} cases, {len(shapes['buckets'])} buckets)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
