"""CPU oracle for the MoE expert path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference TorchTurbo's pure-PyTorch
("native") implementation of the MoE expert hot path so that the HIP path can
be checked against it. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker
(or the CPU baseline that is timed); the product package ``torchturbo_amd``
never imports it and has no CPU fallback.

Modules and the reference code they restate (paths relative to the
reference checkout):

* ``native_providers/moe_permutation.py`` —
  ``src/torchturbo/ops/providers/native/moe_permutation.py:17-126``
* ``native_providers/grouped_matmul.py`` —
  ``src/torchturbo/ops/providers/native/grouped_matmul.py:9-56``
* ``native_providers/swiglu.py`` — ``ops/providers/native/swiglu.py:10-24``,
  plus the probability weighting of
  ``src/torchturbo/models/modules/moe/experts.py:181-186``
* ``native_providers/gated_activation.py`` —
  ``ops/providers/native/gated_activation.py:15-68``
* ``native_providers/routing.py`` —
  ``src/torchturbo/models/modules/moe/utils.py:30-80,127-230``
* ``native_providers/grouped_matmul_fp8.py`` and ``fp8.py`` —
  ``scripts/dequant/bailing.py:57-102``, ``scripts/dequant/dequantize.py:62-78``
* ``route_np.py`` — numpy restatement of the packed-row order defined by
  ``src/torchturbo/ops/moe.py:10-46`` (integer work, independent of torch)
* ``layer.py`` — the composition of
  ``src/torchturbo/models/modules/moe/moe_layer.py:149-183`` with the EP=1
  dispatcher stages of ``token_dispatcher.py:125-236`` and
  ``experts.py:188-266``
* ``dense.py`` — the per-token loop of
  ``tests/models/test_moe_probability_weighting.py:134-165``

Pinning (what checks each function beyond its own restatement) is listed in
each module's docstring; ``tests/test_oracle_*.py`` hold the checks.
"""
