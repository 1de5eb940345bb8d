"""Availability probe shared by the HIP providers (no op classes here)."""

from __future__ import annotations

import torch


def hip_available() -> bool:
    """True on a PyTorch-ROCm build with a visible GPU. Never raises."""
    try:
        return torch.version.hip is not None and torch.cuda.is_available()
    except Exception:  # noqa: BLE001 - availability probes must not raise
        return False
