"""MI355X-native MoE expert path with TorchTurbo's op-provider and MoELayer API.

* ``torchturbo_amd.dispatch`` — op registry, policy dispatcher and the
  process-wide ``ops`` proxy (the drop-in boundary);
* ``torchturbo_amd.moe`` — ``MoELayer`` / ``TopKRouter`` / ``GroupedMLP``
  (and the FP8 expert variant), all routed through ``ops``;
* ``torchturbo_amd.providers.hip`` — providers backed by hand-written gfx950
  HIP kernels, reached through the C-ABI library ``libtorchturbo_moe.so``
  (``include/torchturbo_moe.h``).
"""

from __future__ import annotations

__version__ = "0.1.0"

from .dispatch import OpPolicy, get_or_create_ops, ops  # noqa: E402
from .runtime import get_device_runtime  # noqa: E402


def init_ops(policy: OpPolicy = OpPolicy.AUTO, overrides=None, device_runtime=None):
    """Create (or fetch) the process dispatcher for the detected device."""
    return get_or_create_ops(device_runtime=device_runtime or get_device_runtime(),
                             default_policy=policy, overrides=overrides)


__all__ = ["OpPolicy", "get_device_runtime", "get_or_create_ops", "init_ops", "ops"]
