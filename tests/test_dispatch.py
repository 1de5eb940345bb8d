"""Op registry / dispatcher policy semantics (CPU).

Mirrors the selection rules of ``src/torchturbo/ops/{registry,dispatcher,ops}.py``
(see ``tests/ops/test_dispatch.py`` of the reference for the same behaviours):
ranking, policy filtering, fallback only under ``auto``, explicit
implementations and overrides never falling back, unresolved ops logged,
process-wide dispatcher reuse rules, facade validation errors.
"""

from __future__ import annotations

import sys
import types

import pytest
import torch

from torchturbo_amd.dispatch import (
    OpDispatcher,
    OpImpl,
    OpImplKind,
    OpPolicy,
    OpRegistry,
    OpSpec,
    add_provider_package,
    get_or_create_ops,
    remove_provider_package,
)
from torchturbo_amd.runtime import CpuRuntime, CudaRuntime, TurboDevice


def make_provider_module(name, registry, impls):
    """A throwaway provider module with OpImpl classes registered in ``registry``."""
    mod = types.ModuleType(name)
    for impl_name, op_name, kind, prio, devices, available, result in impls:
        spec = OpSpec(op_name=op_name, impl_name=impl_name, kind=kind, priority=prio,
                      devices=devices)
        registry.register(spec)

        def call(self, *a, _r=result, **kw):
            return _r

        cls = type(impl_name, (OpImpl,), {
            "__call__": call,
            "available": (lambda self, _a=available: _a),
            "__module__": name,
        })
        cls.__op_spec__ = spec
        setattr(mod, impl_name, cls)
    sys.modules[name] = mod
    return mod


@pytest.fixture
def fake_registry(monkeypatch):
    reg = OpRegistry()
    make_provider_module("fake_providers_mod", reg, [
        ("native_x", "opx", OpImplKind.NATIVE, 0, (), True, "native"),
        ("custom_x", "opx", OpImplKind.CUSTOM, 200, (TurboDevice.CUDA,), False, "custom"),
        ("custom_x_cpu", "opx", OpImplKind.CUSTOM, 5, (TurboDevice.CPU,), True, "custom_cpu"),
        ("native_y", "opy", OpImplKind.NATIVE, 0, (), True, "y"),
    ])
    add_provider_package("fake_providers_mod")
    yield reg
    remove_provider_package("fake_providers_mod")
    sys.modules.pop("fake_providers_mod", None)


def test_spec_validation():
    with pytest.raises(ValueError):
        OpSpec(op_name="", impl_name="a")
    with pytest.raises(ValueError, match="reserved"):
        OpSpec(op_name="a", impl_name="auto")
    with pytest.raises(TypeError):
        OpSpec(op_name="a", impl_name="b", kind="native")
    reg = OpRegistry()
    reg.register(OpSpec(op_name="a", impl_name="b"))
    with pytest.raises(ValueError, match="already registered"):
        reg.register(OpSpec(op_name="c", impl_name="b"))


def test_ranking_priority_device_kind():
    reg = OpRegistry()
    for spec in (OpSpec("o", "n0", OpImplKind.NATIVE, 0, ()),
                 OpSpec("o", "c0", OpImplKind.CUSTOM, 0, ()),
                 OpSpec("o", "d0", OpImplKind.NATIVE, 0, (TurboDevice.CPU,)),
                 OpSpec("o", "hi", OpImplKind.NATIVE, 9, ())):
        reg.register(spec)
    assert [s.impl_name for s in reg.list()] == ["hi", "d0", "c0", "n0"]


def test_auto_falls_back_past_unavailable(fake_registry):
    d = OpDispatcher(device_runtime=CudaRuntime(), registry=fake_registry)
    assert d.opx() == "native"  # custom_x (CUDA) unavailable -> fallback
    assert "fallback" in d.log_ops_selection()


def test_custom_policy_never_falls_back_to_native(fake_registry):
    d = OpDispatcher(device_runtime=CudaRuntime(), registry=fake_registry,
                     default_policy=OpPolicy.CUSTOM)
    with pytest.raises(RuntimeError, match="unavailable"):
        d.opx()
    assert "opx" in d.unresolved_ops


def test_native_policy_ignores_available_custom(fake_registry):
    d = OpDispatcher(device_runtime=CpuRuntime(), registry=fake_registry,
                     default_policy=OpPolicy.NATIVE)
    assert d.opx() == "native"
    d2 = OpDispatcher(device_runtime=CpuRuntime(), registry=fake_registry)
    assert d2.opx() == "custom_cpu"


def test_explicit_impl_and_override_never_fall_back(fake_registry):
    d = OpDispatcher(device_runtime=CudaRuntime(), registry=fake_registry)
    with pytest.raises(RuntimeError, match="custom_x"):
        d.opx(impl="custom_x")
    with pytest.raises(RuntimeError, match="registered for op"):
        d.opx(impl="native_y")
    with pytest.raises(RuntimeError, match="Invalid override"):
        OpDispatcher(device_runtime=CudaRuntime(), registry=fake_registry,
                     overrides={"opx": "custom_x"})
    d3 = OpDispatcher(device_runtime=CpuRuntime(), registry=fake_registry,
                      overrides={"opx": "native_x"})
    assert d3.opx() == "native"
    with pytest.raises(RuntimeError, match="does not support"):
        d.opx(impl="custom_x_cpu")


def test_unknown_op_attribute_error(fake_registry):
    d = OpDispatcher(device_runtime=CpuRuntime(), registry=fake_registry)
    with pytest.raises(AttributeError):
        d.no_such_op
    with pytest.raises(AttributeError):
        d._private


def test_policy_type_and_override_types():
    from torchturbo_amd.dispatch import registry
    with pytest.raises(TypeError):
        OpDispatcher(device_runtime=CpuRuntime(), registry=registry, default_policy="auto")
    with pytest.raises(TypeError):
        OpDispatcher(device_runtime=CpuRuntime(), registry=registry, overrides={"a": 1})


def test_process_dispatcher_reuse_rules(process_ops):
    d = process_ops(CpuRuntime(), OpPolicy.NATIVE, oracle=True)
    assert get_or_create_ops(device_runtime=CpuRuntime(), default_policy=OpPolicy.NATIVE) is d
    with pytest.raises(RuntimeError, match="incompatible"):
        get_or_create_ops(device_runtime=CpuRuntime(), default_policy=OpPolicy.AUTO)
    with pytest.raises(RuntimeError, match="incompatible"):
        get_or_create_ops(device_runtime=CudaRuntime(), default_policy=OpPolicy.NATIVE)


def test_facade_validation_errors(oracle_ops):
    tokens = torch.ones(2, 1)
    # tests/ops/test_moe_permutation_contract.py:437-445
    with pytest.raises(ValueError, match="same top-k"):
        oracle_ops.moe_permutation(tokens, torch.tensor([[True, True], [False, False]]))
    with pytest.raises(ValueError, match="token dropping"):
        oracle_ops.moe_permutation(tokens, torch.ones(2, 2, dtype=torch.bool), num_out_tokens=3)
    with pytest.raises(ValueError, match="input device"):
        oracle_ops.moe_sort_chunks(tokens, torch.tensor([1, 1], device="meta"),
                                   torch.tensor([1, 0]))


def test_product_has_no_cpu_provider():
    """Without the oracle attached, a CPU dispatcher resolves no MoE op: the
    product ships only HIP providers and never falls back to the CPU."""
    import oracle.native_providers.moe_permutation  # noqa: F401  (specs in the registry)
    from torchturbo_amd.dispatch import registry
    remove_provider_package("oracle.native_providers")
    d = OpDispatcher(device_runtime=CpuRuntime(), registry=registry)
    for op in ("moe_permutation", "moe_unpermutation", "grouped_matmul", "swiglu_probs",
               "gated_activation_probs", "router_loss_stats"):
        with pytest.raises(RuntimeError, match="No implementation"):
            d._dispatch(op)


def test_hip_providers_registered_for_cuda_only():
    import torchturbo_amd.providers.hip.grouped_matmul  # noqa: F401
    import torchturbo_amd.providers.hip.moe_permutation  # noqa: F401
    import torchturbo_amd.providers.hip.routing  # noqa: F401
    import torchturbo_amd.providers.hip.swiglu  # noqa: F401
    from torchturbo_amd.dispatch import registry
    hip = [s for s in registry.list() if s.impl_name.startswith("hip_")]
    assert {s.op_name for s in hip} >= {"moe_permutation", "moe_unpermutation", "moe_sort_chunks",
                                        "grouped_matmul", "grouped_matmul_fp8", "swiglu",
                                        "swiglu_probs", "topk_softmax_with_capacity",
                                        "gated_activation", "gated_activation_probs",
                                        "router_loss_stats"}
    assert all(s.devices == (TurboDevice.CUDA,) and s.kind == OpImplKind.CUSTOM
               and s.priority > 100 for s in hip)



def test_one_impl_name_defined_by_two_classes_is_an_error():
    """Two provider classes carrying the same impl_name (ops/dispatcher.py:77-97):
    building a dispatcher over both modules raises ValueError naming both."""
    reg = OpRegistry()
    make_provider_module("fake_dup_a", reg, [("dup_impl", "opd", OpImplKind.NATIVE, 0, (), True, 1)])
    make_provider_module("fake_dup_b", reg, [("dup_impl", "opd", OpImplKind.NATIVE, 0, (), True, 2)])
    add_provider_package("fake_dup_a")
    add_provider_package("fake_dup_b")
    try:
        with pytest.raises(ValueError, match="defined by both fake_dup_a.dup_impl and fake_dup_b.dup_impl"):
            OpDispatcher(device_runtime=CpuRuntime(), registry=reg)
    finally:
        remove_provider_package("fake_dup_a")
        remove_provider_package("fake_dup_b")
        sys.modules.pop("fake_dup_a", None)
        sys.modules.pop("fake_dup_b", None)
