"""Loading HF block-FP8 expert weights (e4m3 ``.weight`` + ``.weight_scale_inv``)
straight into ``Fp8GroupedMLP`` (``moe/fp8_checkpoint.py``), against the
reference's offline path: dequantise each projection (``scripts/dequant/bailing.py:57-102``,
restated in ``oracle/fp8.py``), assemble ``weight1 = cat(gate, up).T`` /
``weight2 = down.T`` (``models/weight_converter.py:417-449``) and run the bf16 experts."""

from __future__ import annotations

import json

import pytest
import torch
import torch.nn.functional as F
from safetensors.torch import save_file

from oracle import fp8 as o_fp8
from torchturbo_amd.dispatch import OpPolicy
from torchturbo_amd.moe import Fp8GroupedMLP, GroupedMLP, MoEConfig, load_fp8_experts
from torchturbo_amd.runtime import CpuRuntime

PREFIX = "model.layers.3.mlp.experts"


def make_checkpoint(E, H, Fi, scale_dtype=torch.bfloat16, seed=0, first=0):
    g = torch.Generator().manual_seed(seed)
    tensors, deq = {}, {}
    for i in range(first, first + E):
        for proj, shape in (("gate_proj", (Fi, H)), ("up_proj", (Fi, H)), ("down_proj", (H, Fi))):
            w = torch.randn(*shape, generator=g) * 0.02
            q, s = o_fp8.quantize_blockwise(w, scale_dtype)
            key = f"{PREFIX}.{i}.{proj}"
            tensors[key + ".weight"] = q
            tensors[key + ".weight_scale_inv"] = s
            deq[(i, proj)] = o_fp8.dequantize_weight(q, s)
    return tensors, deq


def write_sharded(tmp_path, tensors):
    keys = sorted(tensors)
    half = len(keys) // 2
    weight_map = {}
    for n, part in enumerate((keys[:half], keys[half:])):
        name = f"model-{n + 1:05d}-of-00002.safetensors"
        save_file({k: tensors[k].contiguous() for k in part}, str(tmp_path / name))
        weight_map.update({k: name for k in part})
    with open(tmp_path / "model.safetensors.index.json", "w") as f:
        json.dump({"metadata": {}, "weight_map": weight_map}, f)
    return tmp_path


def fp8_module(E, H, Fi):
    cfg = MoEConfig(hidden_size=H, moe_ffn_hidden_size=Fi, gated_linear_unit=True,
                    activation_func=F.silu, params_dtype=torch.bfloat16)
    return Fp8GroupedMLP(E, False, cfg), cfg


@pytest.mark.parametrize("scale_dtype", [torch.bfloat16, torch.float32])
def test_fp8_experts_load_bit_exact_from_sharded_safetensors(tmp_path, scale_dtype):
    E, H, Fi = 3, 256, 128
    tensors, deq = make_checkpoint(E, H, Fi, scale_dtype)
    mod, _ = fp8_module(E, H, Fi)
    load_fp8_experts(mod, write_sharded(tmp_path, tensors), PREFIX)
    assert mod.s1.dtype == scale_dtype and mod.s2.dtype == scale_dtype
    for e in range(E):
        k = f"{PREFIX}.{e}"
        q_gu = torch.cat([tensors[k + ".gate_proj.weight"], tensors[k + ".up_proj.weight"]])
        s_gu = torch.cat([tensors[k + ".gate_proj.weight_scale_inv"],
                          tensors[k + ".up_proj.weight_scale_inv"]])
        assert torch.equal(mod.q1[e].view(torch.uint8), q_gu.view(torch.uint8))
        assert torch.equal(mod.s1[e], s_gu)
        assert torch.equal(mod.q2[e].view(torch.uint8),
                           tensors[k + ".down_proj.weight"].view(torch.uint8))
        assert torch.equal(mod.s2[e], tensors[k + ".down_proj.weight_scale_inv"])
        # master weights: the reference's dequantised BF16 weights, bit for bit
        assert torch.equal(mod.master1[e], torch.cat([deq[(e, "gate_proj")], deq[(e, "up_proj")]]))
        assert torch.equal(mod.master2[e], deq[(e, "down_proj")])


def test_loaded_fp8_experts_match_reference_bf16_assembly(process_ops):
    process_ops(CpuRuntime(), OpPolicy.NATIVE, oracle=True)
    E, H, Fi = 2, 256, 128
    tensors, deq = make_checkpoint(E, H, Fi, seed=1, first=4)
    mod, cfg = fp8_module(E, H, Fi)
    load_fp8_experts(mod, tensors, PREFIX, first_expert=4)
    ref = GroupedMLP(E, False, cfg)
    with torch.no_grad():  # weight_converter.py:417-449
        ref.weight1.copy_(torch.cat([torch.cat([deq[(4 + e, "gate_proj")], deq[(4 + e, "up_proj")]]).T
                                     for e in range(E)]))
        ref.weight2.copy_(torch.cat([deq[(4 + e, "down_proj")].T for e in range(E)]))
    g = torch.Generator().manual_seed(2)
    counts = torch.tensor([5, 9])
    x = torch.randn(14, H, generator=g).to(torch.bfloat16)
    p = torch.rand(14, generator=g)
    got, _ = mod(x, counts, p)
    want, _ = ref(x, counts, p)
    torch.testing.assert_close(got, want, rtol=1e-2, atol=1e-3)


def test_fp8_loader_rejects_bad_tensors():
    E, H, Fi = 1, 256, 128
    tensors, _ = make_checkpoint(E, H, Fi)
    mod, _ = fp8_module(E, H, Fi)
    k = f"{PREFIX}.0.up_proj"
    bad = dict(tensors)
    bad[k + ".weight"] = tensors[k + ".weight"].float()
    with pytest.raises(ValueError, match="expected FP8 E4M3"):
        load_fp8_experts(mod, bad, PREFIX)
    bad = dict(tensors)
    bad[k + ".weight_scale_inv"] = tensors[k + ".weight_scale_inv"][:, :1]
    with pytest.raises(ValueError, match="does not match expected"):
        load_fp8_experts(mod, bad, PREFIX)
    bad = dict(tensors)
    bad[k + ".weight_scale_inv"] = tensors[k + ".weight_scale_inv"].half()
    with pytest.raises(ValueError, match="expected BF16 or FP32"):
        load_fp8_experts(mod, bad, PREFIX)
    bad = {key: v for key, v in tensors.items() if not key.startswith(f"{PREFIX}.0.down_proj")}
    with pytest.raises(KeyError, match="down_proj"):
        load_fp8_experts(mod, bad, PREFIX)
