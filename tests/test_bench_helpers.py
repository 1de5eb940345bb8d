"""CPU checks of bench.py's bookkeeping (no GPU): the per-GEMM breakdown of the
grouped-GEMM launches recorded in one layer step's launch order."""
import importlib.util
import pathlib
import types

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_mod", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _w(M=1024, H=256, F=128):
    return types.SimpleNamespace(routed_rows=M, hidden=H, ffn=F)


def _step(t):
    return [("tt_gmm_fwd_gather", t[0]), ("tt_gmm_fwd", t[1]), ("tt_gmm_dgrad_gather", t[2]),
            ("tt_gmm_wgrad_gather", t[3]), ("tt_gmm_dgrad", t[4]), ("tt_gmm_wgrad_gather", t[5])]


def test_per_gemm_means_and_flops(bench):
    w = _w()
    order = _step([1.0, 0.5, 0.25, 0.5, 1.0, 2.0]) + _step([3.0, 0.5, 0.75, 0.5, 1.0, 2.0])
    out = bench.per_gemm(w, order, 2)
    assert list(out) == list(bench.GEMM_KINDS)
    assert out["fc1_fwd"] == {"entry": "tt_gmm_fwd_gather", "us": 2000.0,
                              "tflops": round(2.0 * 1024 * 256 * 256 / 2000.0 / 1e6, 1)}
    assert out["fc2_dgrad"]["us"] == 500.0
    fc2 = 2.0 * 1024 * 128 * 256
    assert out["fc2_wgrad"]["tflops"] == round(fc2 / 500.0 / 1e6, 1)


def test_per_gemm_rejects_other_launch_orders(bench):
    w = _w()
    good = _step([1.0] * 6)
    assert bench.per_gemm(w, good[:5], 1) is None          # a launch missing
    swapped = [good[1], good[0]] + good[2:]
    assert bench.per_gemm(w, swapped[:2] + [good[3], good[2]] + good[4:], 1) is None  # wgrad before dgrad
    mixed = good + _step([1.0] * 6)
    mixed[6] = ("tt_gmm_fwd", 1.0)                          # fc1 fwd entry differs between steps
    assert bench.per_gemm(w, mixed, 2) is None
    assert bench.per_gemm(w, [], 0) is None
