"""kvpath.kelpie_adapter against stand-ins of kelpie's registry interface (the reference's op.py
`Op.register`, backends.py `declare_backend` / `BACKENDS`, devices.py `CUDA_ARCH_DEFAULTS`),
built here in sys.modules: kelpie itself needs Python >= 3.11 and is not installed."""

from __future__ import annotations

import sys
import types

import pytest


class _Op:
    """The part of kelpie's Op the adapter uses (op.py:51-94)."""

    def __init__(self) -> None:
        self.impls: dict[str, tuple] = {}

    def register(self, impl, *, source=None, backend=None, predicate=None):
        assert impl not in self.impls, f"impl {impl!r} registered twice"

        def decorate(fn):
            self.impls[impl] = (fn, backend if backend is not None else impl, source, predicate)
            return fn

        return decorate


@pytest.fixture()
def fake_kelpie(monkeypatch):
    backends = types.ModuleType("kelpie_models.kernels.backends")
    backends.BACKENDS = {}

    def declare_backend(name, *, package, min_version=None, max_version=None, extra=None):
        assert name not in backends.BACKENDS
        backends.BACKENDS[name] = (package, extra)

    backends.declare_backend = declare_backend
    devices = types.ModuleType("kelpie_models.kernels.devices")
    devices.CUDA_ARCH_DEFAULTS = {(8, 0): {"paged_attention": "vllm_triton"}}
    pa = types.ModuleType("kelpie_models.kernels.ops.paged_attention")
    pa.paged_attention = _Op()
    ops = types.ModuleType("kelpie_models.kernels.ops")
    ops.paged_attention = pa.paged_attention  # kelpie's ops package exports the op object
    mods = {
        "kelpie_models": types.ModuleType("kelpie_models"),
        "kelpie_models.kernels": types.ModuleType("kelpie_models.kernels"),
        "kelpie_models.kernels.backends": backends,
        "kelpie_models.kernels.devices": devices,
        "kelpie_models.kernels.ops": ops,
        "kelpie_models.kernels.ops.paged_attention": pa,
    }
    for name, mod in mods.items():
        monkeypatch.setitem(sys.modules, name, mod)
    return backends, devices, pa


def test_register_plugs_into_the_registry(fake_kelpie) -> None:
    from kvpath import kelpie_adapter

    backends, devices, pa = fake_kelpie
    kelpie_adapter.register()
    fn, backend, source, predicate = pa.paged_attention.impls["mi355x"]
    assert fn is kelpie_adapter.mi355x_paged_attention
    assert backend == "kvpath" and backends.BACKENDS["kvpath"][0] == "kvpath"
    assert "gfx950" in source and predicate is None
    assert devices.CUDA_ARCH_DEFAULTS[(9, 5)] == {"paged_attention": "mi355x"}
    assert devices.CUDA_ARCH_DEFAULTS[(8, 0)] == {"paged_attention": "vllm_triton"}
    kelpie_adapter.register()  # idempotent
    assert list(pa.paged_attention.impls) == ["mi355x"]


def test_register_without_default(fake_kelpie) -> None:
    from kvpath import kelpie_adapter

    _, devices, pa = fake_kelpie
    kelpie_adapter.register(default=False)
    assert "mi355x" in pa.paged_attention.impls
    assert (9, 5) not in devices.CUDA_ARCH_DEFAULTS


def test_impl_refuses_cpu_like_the_op(fake_kelpie) -> None:
    """The impl is the kvpath op: CPU tensors raise (there is no CPU path)."""
    import torch

    from kvpath import kelpie_adapter
    from workloads import Batch, step_args

    args = step_args(Batch(entries=((3, 1),), tokens=1, reqs=1, heads=4, kv_heads=2,
                           head_dim=32, block=4), "cpu", torch.bfloat16)
    with pytest.raises(RuntimeError, match="no CPU path"):
        kelpie_adapter.mi355x_paged_attention(*args)
