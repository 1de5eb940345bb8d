"""Shared fixtures. GPU tests are marked ``gpu`` and need a ROCm device."""

from __future__ import annotations

import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm) GPU and the built HIP library")


@pytest.fixture
def oracle_ops():
    """CPU dispatcher whose providers are the oracle's native restatements."""
    from torchturbo_amd.dispatch import OpDispatcher, OpPolicy, add_provider_package, registry
    from torchturbo_amd.runtime import CpuRuntime

    add_provider_package("oracle.native_providers")
    return OpDispatcher(device_runtime=CpuRuntime(), registry=registry, default_policy=OpPolicy.NATIVE)


@pytest.fixture
def hip_ops():
    """GPU dispatcher with the product's providers only (no oracle attached)."""
    from torchturbo_amd.dispatch import OpDispatcher, OpPolicy, registry, remove_provider_package
    from torchturbo_amd.runtime import CudaRuntime

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    remove_provider_package("oracle.native_providers")
    ops = OpDispatcher(device_runtime=CudaRuntime(), registry=registry, default_policy=OpPolicy.CUSTOM)
    return ops


@pytest.fixture
def process_ops(monkeypatch):
    """Install a fresh process-wide dispatcher; yields a setter (runtime, policy)."""
    import importlib

    from torchturbo_amd.dispatch import add_provider_package, get_or_create_ops, remove_provider_package

    # the package re-exports the ``ops`` proxy under the module's name
    ops_mod = importlib.import_module("torchturbo_amd.dispatch.ops")

    monkeypatch.setattr(ops_mod, "_OPS", None)

    def make(runtime, policy, oracle: bool = False):
        """``oracle=True`` attaches the CPU oracle's native providers."""
        if oracle:
            add_provider_package("oracle.native_providers")
        else:
            remove_provider_package("oracle.native_providers")
        ops_mod._OPS = None  # each call installs a fresh dispatcher
        return get_or_create_ops(device_runtime=runtime, default_policy=policy)

    yield make
    ops_mod._OPS = None


def rel_errors(actual: torch.Tensor, expected: torch.Tensor) -> tuple[float, float]:
    """(max |a-b| / max |b|, mean |a-b| / mean |b|) in float64."""
    a = actual.detach().double().cpu()
    b = expected.detach().double().cpu()
    diff = (a - b).abs()
    denom_max = b.abs().max().item() if b.numel() else 0.0
    denom_mean = b.abs().mean().item() if b.numel() else 0.0
    mx = diff.max().item() / denom_max if denom_max > 0 else diff.max().item() if diff.numel() else 0.0
    mean = diff.mean().item() / denom_mean if denom_mean > 0 else diff.mean().item() if diff.numel() else 0.0
    return mx, mean


def assert_bf16_close(actual, expected, max_rel=2e-2, mean_rel=2e-3, what=""):
    """The path's tolerance: normwise max relative error <= 2e-2, mean <= 2e-3."""
    mx, mean = rel_errors(actual, expected)
    assert mx <= max_rel and mean <= mean_rel, f"{what}: max_rel={mx:.3e} mean_rel={mean:.3e}"
