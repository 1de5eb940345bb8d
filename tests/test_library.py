"""The C-ABI library: builds, loads without a GPU, exports every declared
entry point, and rejects invalid arguments before touching the device (CPU)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from torchturbo_amd import _lib as L
from torchturbo_amd.build import library_path

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols() -> set[str]:
    names = set()
    for header in (ROOT / "include").glob("*.h"):
        text = header.read_text()
        names.update(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(tt_\w+)\s*\(", text, re.M))
    return names


@pytest.fixture(scope="module")
def lib():
    if not library_path().exists():
        pytest.fail("HIP library not built; run `python -m torchturbo_amd.build`")
    return L.load()


def test_header_declares_the_bound_prototypes():
    declared = declared_symbols()
    assert declared, "no tt_* declarations found in include/*.h"
    assert declared == set(L._PROTOS), declared ^ set(L._PROTOS)


def test_library_exports_every_declared_symbol(lib):
    raw = ctypes.CDLL(str(library_path()))
    for name in sorted(declared_symbols()):
        assert hasattr(raw, name), name
    assert lib.tt_abi_version() == L.ABI_VERSION


@pytest.mark.parametrize("name,args,msg", [
    ("tt_router_topk_fwd", (None, 9, 4, 8, 2, 0, 0, None, 0, 0, 0.0, None, None, None, None, None),
     "dtype"),
    ("tt_router_topk_fwd", (None, 0, 4, 2000, 2, 0, 0, None, 0, 0, 0.0, None, None, None, None,
                            None), "num_experts"),
    ("tt_router_topk_fwd", (None, 0, 4, 10, 2, 0, 0, None, 3, 1, 0.0, None, None, None, None,
                            None), "divisible"),
    ("tt_permute_scatter", (None, 0, 4, 8, 65, None, None, None), "topk"),
    ("tt_unpermute_gather", (None, 7, 4, 8, 2, None, None, None, 0, 1, None, None), "dtype"),
    ("tt_swiglu_fwd", (None, 0, -1, 8, None, 0, None, None), "negative"),
    ("tt_gmm_fwd", (None, None, 1, 16, 12, 16, 2, 0, None, None, None), "multiples of 8"),
    ("tt_gmm_fwd", (None, None, 5, 16, 16, 16, 2, 0, None, None, None), "dtype"),
    ("tt_gmm_fwd", (None, None, 1, 16, 16, 16, 0, 0, None, None, None), "num_experts"),
    ("tt_gmm_fp8_fwd", (None, None, None, 2, 16, 16, 16, 2, None, None, None), "scales"),
    ("tt_gmm_fwd_gather", (None, 8, None, None, 1, 16, 128, 16, 2, 0, None, None, None),
     "row map"),
    ("tt_gmm_fwd_gather", (None, 8, None, None, 0, 16, 128, 16, 2, 0, None, None, None), "dtype"),
    ("tt_route_index", (None, 4, 2, 8, None, 0, None, None, None, None, None, 0, None),
     "workspace"),
    ("tt_sort_chunks", (None, 0, 4, 4, None, None, 5000, None, 0, None, None, None), "4096"),
])
def test_invalid_arguments_fail_before_any_launch(lib, name, args, msg):
    with pytest.raises(ValueError, match=msg):
        L.call(name, *args)


def test_empty_problems_are_no_ops(lib):
    # zero tokens: nothing is launched and the call succeeds
    L.call("tt_permute_scatter", None, 1, 0, 8, 2, None, None, None)
    L.call("tt_unpermute_gather", None, 1, 0, 8, 2, None, None, None, 0, 1, None, None)
    L.call("tt_swiglu_fwd", None, 1, 0, 8, None, 0, None, None)
    L.call("tt_router_topk_fwd", None, 0, 0, 8, 2, 0, 0, None, 0, 0, 0.0, None, None, None,
           None, None)
    L.call("tt_packed_probs_bwd", None, 0, 0, 2, 8, None, None, None, None)


def test_shape_queries_answer_without_a_gpu(lib):
    """The launch-choice queries are host arithmetic: the benchmark layers' shapes."""
    bf = L.TT_BF16
    wp = lib.tt_gmm_wgrad_persistent
    # Qwen3 fc1 (48 output tiles per expert) and fc2 (24), 1024 rows per expert on average
    assert wp(bf, 131072, 2048, 1536, 128, 0) == 0
    assert wp(bf, 131072, 768, 2048, 128, 0) == 0
    # the boundary: 16 x 32 tiles per expert are persistent, 16 x 31 are not
    assert wp(bf, 8192, 4096, 8192, 8, 0) == 1
    assert wp(bf, 8192, 4096, 7936, 8, 0) == 0
    assert wp(bf, 8192, 8192, 4096, 8, 1) == 1
    # short reductions (DeepSeek-V3: 128 rows per expert) and Mixtral's large grids
    assert wp(bf, 32768, 7168, 4096, 256, 1) == 1
    assert wp(bf, 32768, 2048, 7168, 256, 1) == 1
    assert wp(bf, 16384, 4096, 28672, 8, 0) == 1
    assert wp(bf, 16384, 14336, 4096, 8, 0) == 1
    # fp32 takes its own kernel; invalid sizes are never persistent
    assert wp(L.TT_F32, 131072, 2048, 1536, 128, 0) == 0
    assert wp(bf, -1, 2048, 1536, 128, 0) == 0 and wp(bf, 1024, 2048, 1536, 0, 0) == 0
    gs = lib.tt_gmm_gather_supported
    # the Qwen3 layer's four gathering launches are taken; more experts than the LDS
    # schedule holds are not; fp32 is not
    assert gs(0, bf, 16384, 131072, 2048, 1536, 128) == 1
    assert gs(1, bf, 16384, 131072, 768, 2048, 128) == 1
    assert gs(2, bf, 16384, 131072, 2048, 1536, 128) == 1
    assert gs(3, bf, 16384, 131072, 768, 2048, 128) == 1
    assert gs(0, bf, 16384, 1048576, 2048, 1536, 1024) == 0
    assert gs(0, L.TT_F32, 16384, 131072, 2048, 1536, 128) == 0
    # gathering weight gradients take sources of fewer than 2^24 rows (24-bit offsets)
    assert gs(2, bf, (1 << 24) - 1, 1 << 24, 64, 64, 8) == 1
    assert gs(2, bf, 1 << 24, 1 << 24, 64, 64, 8) == 0
