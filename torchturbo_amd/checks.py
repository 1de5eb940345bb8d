"""Input checks that need the host to read device memory (off by default).

The HIP providers never synchronise the host on their own: routing counts,
split sizes and row maps stay on the device. Inputs that break the op
contracts are still handled without a fault (a rejected routing slot gets row
-1 and contributes nothing; see ``tt_route_index``), but the reference's
native path raises on them (``ops/moe.py:62-65``, ``native/moe_permutation.py:52-56``,
``torch.split`` in ``native/moe_permutation.py:117-119``). With checks on, the
providers read the device-side verdicts back and raise ``ValueError`` the
same way, at the price of one host synchronisation per checked call.

Turn on with ``TORCHTURBO_CHECK_INPUTS=1`` in the environment or
``torchturbo_amd.checks.set_enabled(True)``.
"""

from __future__ import annotations

import contextlib
import os

_ENABLED = os.environ.get("TORCHTURBO_CHECK_INPUTS", "0") not in ("", "0")


def enabled() -> bool:
    return _ENABLED


def set_enabled(flag: bool) -> None:
    global _ENABLED
    _ENABLED = bool(flag)


@contextlib.contextmanager
def checking(flag: bool = True):
    """``with checking(): ...`` turns the checks on (or off) for a block."""
    global _ENABLED
    saved = _ENABLED
    _ENABLED = bool(flag)
    try:
        yield
    finally:
        _ENABLED = saved


__all__ = ["checking", "enabled", "set_enabled"]
