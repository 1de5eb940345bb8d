"""Device runtime for the MoE expert path.

Mirrors the reference's ``TurboDevice`` / ``DeviceRuntime`` surface
(``src/torchturbo/runtime/base.py:33-138``, ``runtime/runtime.py:9-61``)
for the two devices this build runs on: a PyTorch-ROCm GPU (reported as
``cuda``, exactly as the reference's ``CudaRuntime`` sees it on ROCm,
``runtime/cuda.py:73-90``) and the host CPU.
"""

from __future__ import annotations

import contextlib
from enum import Enum

import torch


class TurboDevice(str, Enum):
    """Runtime devices (``runtime/base.py:33-38``)."""

    CUDA = "cuda"
    NPU = "npu"
    CPU = "cpu"

    def __str__(self) -> str:  # behave like the reference's StrEnum
        return self.value


class DeviceRuntime:
    turbo_device: TurboDevice
    dist_backend: str

    @property
    def device(self) -> torch.device:
        return torch.device(self.turbo_device.value)

    @property
    def supports_async_streams(self) -> bool:
        return False

    def available(self) -> bool:
        raise NotImplementedError

    def current_stream(self):
        return None

    def new_stream(self):
        return None

    @contextlib.contextmanager
    def stream(self, stream):
        yield

    def synchronize_stream(self, stream) -> None:
        return None

    def synchronize(self) -> None:
        return None


class CudaRuntime(DeviceRuntime):
    """PyTorch-ROCm GPU runtime. Streams are HIP streams at default priority."""

    turbo_device = TurboDevice.CUDA
    dist_backend = "nccl"  # RCCL on ROCm

    @property
    def supports_async_streams(self) -> bool:
        return True

    def available(self) -> bool:
        return torch.cuda.is_available()

    def current_stream(self):
        return torch.cuda.current_stream()

    def new_stream(self):
        if not torch.cuda.is_available():
            return None
        return torch.cuda.Stream()

    def stream(self, stream):
        if stream is None:
            return contextlib.nullcontext()
        return torch.cuda.stream(stream)

    def synchronize_stream(self, stream) -> None:
        if stream is not None:
            stream.synchronize()

    def synchronize(self) -> None:
        torch.cuda.synchronize()


class CpuRuntime(DeviceRuntime):
    turbo_device = TurboDevice.CPU
    dist_backend = "gloo"

    def available(self) -> bool:
        return True


_SELECTED_RUNTIME: DeviceRuntime | None = None


def get_device_runtime() -> DeviceRuntime:
    """Auto-detect GPU then CPU, once per process (``runtime/runtime.py:46-61``)."""
    global _SELECTED_RUNTIME
    if _SELECTED_RUNTIME is None:
        cuda = CudaRuntime()
        _SELECTED_RUNTIME = cuda if cuda.available() else CpuRuntime()
    return _SELECTED_RUNTIME


def set_device_runtime(runtime: DeviceRuntime | None) -> None:
    global _SELECTED_RUNTIME
    _SELECTED_RUNTIME = runtime


__all__ = [
    "CpuRuntime",
    "CudaRuntime",
    "DeviceRuntime",
    "TurboDevice",
    "get_device_runtime",
    "set_device_runtime",
]
