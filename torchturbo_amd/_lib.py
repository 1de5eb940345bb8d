"""ctypes binding of the C-ABI kernel library (``include/torchturbo_moe.h``).

The library is loaded lazily from ``torchturbo_amd/_lib/libtorchturbo_moe.so``;
a missing library raises ``RuntimeError`` (there is no fallback path). Calls
pass raw device pointers and enqueue on PyTorch's current HIP stream.
"""

from __future__ import annotations

import ctypes
from ctypes import c_float, c_int, c_int32, c_int64, c_size_t, c_void_p

import torch

from .build import library_path

TT_F32, TT_BF16, TT_F16, TT_F8E4M3, TT_F64 = 0, 1, 2, 3, 4
TT_SCORE = {"softmax": 0, "sigmoid": 1, "sqrtsoftplus": 2}

_DTYPES = {
    torch.float32: TT_F32,
    torch.bfloat16: TT_BF16,
    torch.float16: TT_F16,
    torch.float8_e4m3fn: TT_F8E4M3,
    torch.float64: TT_F64,
}

P = c_void_p
I64 = c_int64
I32 = c_int32

# name -> argtypes (all return int status unless listed in _RESTYPES)
_PROTOS: dict[str, list] = {
    "tt_abi_version": [],
    "tt_last_error": [],
    "tt_router_topk_fwd": [P, c_int, I64, I32, I32, I32, I32, P, I32, I32, c_float, P, P, P, P, P],
    "tt_router_topk_bwd": [P, c_int, I64, I32, I32, I32, I32, c_float, P, P, P, P],
    "tt_route_index_workspace": [I64, I32],
    "tt_route_index_rejected_offset": [I64, I32],
    "tt_router_gate_fwd": [P, P, c_int, I64, I64, I32, c_int, I32, I32, I32, P, I32, I32, c_float,
                           P, P, P, P, P, P],
    "tt_router_loss_workspace": [I64, I32],
    "tt_router_loss_fwd": [P, c_int, I64, I32, I32, I32, P, P, P, P, P, c_size_t, P],
    "tt_router_loss_bwd": [P, c_int, I64, I32, I32, P, P, P, P, P],
    "tt_route_index": [P, I64, I32, I32, P, c_int, P, P, P, P, P, c_size_t, P],
    "tt_route_index_noalloc": [P, I64, I32, I32, P, c_int, P, P, P, P, P, P],
    "tt_permute_scatter": [P, c_int, I64, I64, I32, P, P, P],
    "tt_unpermute_gather": [P, c_int, I64, I64, I32, P, P, P, c_int, I32, P, P],
    "tt_unpermute_gather_bwd": [P, P, c_int, I64, I64, I32, P, P, P, c_int, I32, P, P, P],
    "tt_packed_probs_bwd": [P, c_int, I64, I32, I32, P, P, P, P],
    "tt_sort_chunks": [P, c_int, I64, I64, P, P, I32, P, c_int, P, P, P],
    "tt_swiglu_fwd": [P, c_int, I64, I64, P, c_int, P, P],
    "tt_swiglu_bwd": [P, c_int, I64, I64, P, c_int, P, P, P, P],
    "tt_gated_act_fwd": [P, c_int, I64, I64, c_int, c_float, c_int, P, c_int, P, P],
    "tt_gated_act_bwd": [P, c_int, I64, I64, c_int, c_float, c_int, P, c_int, P, P, P, P],
    "tt_gmm_fwd": [P, P, c_int, I64, I64, I64, I32, I32, P, P, P],
    "tt_gmm_dgrad": [P, P, c_int, I64, I64, I64, I32, I32, P, P, P],
    "tt_gmm_wgrad": [P, P, c_int, I64, I64, I64, I32, I32, P, P, P],
    "tt_gmm_fwd_gather": [P, I64, P, P, c_int, I64, I64, I64, I32, I32, P, P, P],
    "tt_gmm_dgrad_gather": [P, I64, P, P, c_int, I64, I64, I64, I32, I32, P, P, P],
    "tt_gmm_wgrad_gather": [P, I64, P, P, I64, P, c_int, I64, I64, I64, I32, I32, P, P, P],
    "tt_gmm_gather_supported": [I32, c_int, I64, I64, I64, I64, I32],
    "tt_gmm_wgrad_persistent": [c_int, I64, I64, I64, I32, I32],
    "tt_gmm_fp8_fwd": [P, P, P, c_int, I64, I64, I64, I32, P, P, P],
    "tt_gmm_fp8_dgrad": [P, P, P, c_int, I64, I64, I64, I32, P, P, P],
}
_RESTYPES = {"tt_last_error": ctypes.c_char_p, "tt_route_index_workspace": c_size_t,
             "tt_route_index_rejected_offset": c_size_t, "tt_router_loss_workspace": c_size_t}
ABI_VERSION = 1

_LIB: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load the kernel library (once) and declare every prototype."""
    global _LIB
    if _LIB is None:
        path = library_path()
        if not path.exists():
            raise RuntimeError(
                f"HIP kernel library {path} is not built; run `python -m torchturbo_amd.build`."
            )
        lib = ctypes.CDLL(str(path))
        for name, argtypes in _PROTOS.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = _RESTYPES.get(name, c_int)
        if lib.tt_abi_version() != ABI_VERSION:
            raise RuntimeError("kernel library ABI version mismatch; rebuild it")
        _LIB = lib
    return _LIB


def is_built() -> bool:
    return library_path().exists()


class KernelTimer:
    """Brackets selected entry points with HIP events on the current stream.

    ``timer.elapsed_ms()`` returns {entry point: (launches, total ms)} after a
    device synchronisation. Used by the benchmark to time the dominant kernel
    on the stream it runs on.
    """

    def __init__(self, names):
        self.names = set(names)
        self.events: list[tuple[str, torch.cuda.Event, torch.cuda.Event]] = []

    def elapsed_ms(self) -> dict[str, tuple[int, float]]:
        torch.cuda.synchronize()
        out: dict[str, tuple[int, float]] = {}
        for name, a, b in self.events:
            n, t = out.get(name, (0, 0.0))
            out[name] = (n + 1, t + a.elapsed_time(b))
        return out


_TIMER: KernelTimer | None = None


def set_timer(timer: KernelTimer | None) -> None:
    global _TIMER
    _TIMER = timer


def call(name: str, *args) -> None:
    """Invoke ``name`` and raise ``RuntimeError`` with the library's message on failure."""
    lib = load()
    timer = _TIMER
    if timer is not None and name in timer.names:
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        rc = getattr(lib, name)(*args)
        b.record()
        timer.events.append((name, a, b))
    else:
        rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.tt_last_error().decode(errors="replace")
        kind = {-1: "invalid argument", -2: "unsupported", -3: "HIP error"}.get(rc, str(rc))
        exc = ValueError if rc == -1 else RuntimeError
        raise exc(f"{name} failed ({kind}): {msg}")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPES[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype for the HIP kernels: {dtype}") from None


def ptr(t: torch.Tensor | None):
    return None if t is None else c_void_p(t.data_ptr())


def stream(device: torch.device | None = None):
    return c_void_p(torch.cuda.current_stream(device).cuda_stream)


def route_index_workspace(num_tokens: int, num_experts: int) -> int:
    return int(load().tt_route_index_workspace(num_tokens, num_experts))


def route_index_rejected_offset(num_tokens: int, num_experts: int) -> int:
    return int(load().tt_route_index_rejected_offset(num_tokens, num_experts))


def router_loss_workspace(num_tokens: int, num_experts: int) -> int:
    return int(load().tt_router_loss_workspace(num_tokens, num_experts))
