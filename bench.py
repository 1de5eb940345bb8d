#!/usr/bin/env python3
"""MoE layer fwd+bwd throughput on one MI355X (HIP kernels through the op API).

One step = routing (top-k softmax) -> permute -> fc1 grouped GEMM -> SwiGLU x
probs -> fc2 grouped GEMM -> unpermute, forward and backward, on one batch of
synthetic inputs already resident in HBM (``MoELayer.forward_with_logits``
with every op served by the HIP providers). On one GPU the layer folds the
permutation into fc1 and the unpermutation's backward into fc2's gradients
(the GEMMs gather token rows through the routing index), when the shapes
allow: the Qwen and varlen layers (Mixtral stays packed). Default workload: the
Qwen3-30B-A3B-shaped layer (16384 tokens, hidden 2048, 128 experts, top-8,
ffn 768, bf16, Zipf-skewed fp32 router logits).

Prints one JSON line with the throughput, the grouped-GEMM roofline (HIP
events around every grouped-GEMM launch on the compute stream) and the CPU
oracle timed on a bounded sample of the same workload.

``--part router`` times the router front end instead: ``TopKRouter`` forward
and backward on the workload's tokens (gating linear fused with the top-k,
aux-loss and z-loss sums, 16-bit router weight, fp32 router dtype).
``--part dense-compare`` times the workload's GEMM shapes through hipBLASLt
beside the grouped kernels (see ``dense_compare``).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16
HBM_PEAK_GBS = 8000.0
GEMM_ENTRIES = ("tt_gmm_fwd", "tt_gmm_dgrad", "tt_gmm_wgrad", "tt_gmm_fwd_gather",
                "tt_gmm_dgrad_gather", "tt_gmm_wgrad_gather", "tt_gmm_fp8_fwd", "tt_gmm_fp8_dgrad")
PERMUTE_ENTRIES = ("tt_permute_scatter", "tt_unpermute_gather")
SWIGLU_ENTRIES = ("tt_swiglu_fwd", "tt_swiglu_bwd")
ROUTER_ENTRIES = ("tt_router_gate_fwd", "tt_router_topk_fwd", "tt_router_topk_bwd",
                  "tt_router_loss_fwd", "tt_router_loss_bwd")


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--workload", default="qwen3_30b_a3b")
    p.add_argument("--part", choices=("layer", "router", "dense-compare"), default="layer",
                   help="layer: the MoE layer step (default); router: the router front end "
                        "only; dense-compare: the workload's GEMM shapes as dense and "
                        "per-expert batched hipBLASLt products (torch.matmul / torch.bmm) "
                        "beside the grouped kernels at uniform loads")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-budget-s", type=float, default=20.0)
    p.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                   help="only run a plain device-to-device copy of BYTES bytes "
                        "(the reference kernel that scales the FETCH_SIZE / WRITE_SIZE "
                        "counters to bytes)")
    return p.parse_args()


def copy_calibration(nbytes, launches=4):
    """A copy of known size: each launch reads and writes exactly ``nbytes``."""
    dev = torch.device("cuda", 0)
    src = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(launches):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "copy", "bytes": nbytes, "launches": launches}), flush=True)


def measured_traffic(workload):
    """HBM bytes per grouped-GEMM launch from the committed counter summary
    ``profiles/gmm_traffic_<workload>.txt`` (line ``bytes_per_launch: N``),
    or None when no such summary exists."""
    path = os.path.join(ROOT, "profiles", f"gmm_traffic_{workload}.txt")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("bytes_per_launch:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def build_layer(w, device):
    import torch.nn.functional as F

    from torchturbo_amd import configs as C
    from torchturbo_amd.moe import Fp8GroupedMLP, GroupedMLP, MoEConfig, MoELayer, MoESubmodules, ModuleSpec

    cfg = MoEConfig(
        hidden_size=w.hidden, num_moe_experts=w.experts, moe_ffn_hidden_size=w.ffn,
        gated_linear_unit=True, activation_func=F.silu, moe_router_topk=w.topk,
        moe_router_pre_softmax=w.pre_softmax, moe_router_score_function=w.score_function,
        moe_router_num_groups=w.num_groups, moe_router_group_topk=w.group_topk,
        moe_router_topk_scaling_factor=w.scaling_factor, params_dtype=w.dtype,
        moe_router_enable_expert_bias=w.expert_bias, perform_initialization=False,
    )
    experts = Fp8GroupedMLP if w.fp8 else GroupedMLP
    layer = MoELayer(cfg, None, submodules=MoESubmodules(experts=ModuleSpec(module=experts)))
    layer = layer.to(device)
    w1, w2 = C.make_weights(w, device=device)
    with torch.no_grad():
        if w.fp8:
            q1, s1 = C.fp8_blocks(w1.transpose(1, 2).contiguous())
            q2, s2 = C.fp8_blocks(w2.transpose(1, 2).contiguous())
            layer.experts.load_quantized(q1, s1, q2, s2)
        else:
            layer.experts.weight1.copy_(w1.reshape(-1, 2 * w.ffn))
            layer.experts.weight2.copy_(w2.reshape(-1, w.hidden))
        bias = C.make_expert_bias(w, device=device)
        if bias is not None:
            layer.router.expert_bias.copy_(bias)
    del w1, w2
    shared = None
    if w.shared_ffn:
        g = torch.Generator(device=device).manual_seed(w.seed + 9)
        mk = lambda *s: torch.empty(*s, device=device).normal_(0, 0.02, generator=g).to(w.dtype)  # noqa: E731
        gate, up, down = (mk(w.shared_ffn, w.hidden), mk(w.shared_ffn, w.hidden),
                          mk(w.hidden, w.shared_ffn))
        for t in (gate, up, down):
            t.requires_grad_()

        def shared(x):
            return F.linear(F.silu(F.linear(x, gate)) * F.linear(x, up), down)
    return layer, shared


def gpu_run(w, steps, warmup):
    from torchturbo_amd import _lib as L
    from torchturbo_amd import configs as C
    from torchturbo_amd.dispatch import OpPolicy, get_or_create_ops
    from torchturbo_amd.runtime import CudaRuntime

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    get_or_create_ops(device_runtime=CudaRuntime(), default_policy=OpPolicy.CUSTOM)
    layer, shared = build_layer(w, dev)
    hidden = C.make_hidden(w, device=dev).requires_grad_()
    logits = C.make_logits(w, device=dev).requires_grad_()
    grad = C.make_grad(w, device=dev)
    params = [p for p in layer.parameters() if p.requires_grad]

    def step():
        for p in params:
            p.grad = None
        hidden.grad = None
        logits.grad = None
        out = layer.forward_with_logits(hidden, logits)
        if shared is not None:
            out = out + shared(hidden)
        out.backward(grad)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    timer = L.KernelTimer(GEMM_ENTRIES + PERMUTE_ENTRIES + SWIGLU_ENTRIES)
    L.set_timer(timer)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    L.set_timer(None)
    kernels = timer.elapsed_ms()
    order = [(n, a.elapsed_time(b)) for n, a, b in timer.events if n in GEMM_ENTRIES]
    return (t1 - t0) * 1e3 / steps, kernels, order


GEMM_KINDS = ("fc1_fwd", "fc2_fwd", "fc2_dgrad", "fc2_wgrad", "fc1_dgrad", "fc1_wgrad")


def per_gemm(w, order, steps):
    """Mean HIP-event time and TFLOP/s of each of the step's six grouped GEMMs,
    told apart by launch order (forward fc1, fc2; backward fc2 dgrad, fc2
    wgrad, fc1 dgrad, fc1 wgrad). None when the launches do not follow it."""
    if steps < 1 or len(order) != 6 * steps:
        return None
    for i, kind in enumerate(GEMM_KINDS):
        names = {n for n, _ in order[i::6]}
        op = kind.split("_")[1]
        if len(names) != 1 or op not in next(iter(names)):
            return None
    M, H, F = w.routed_rows, w.hidden, w.ffn
    out = {}
    for i, kind in enumerate(GEMM_KINDS):
        us = sum(t for _, t in order[i::6]) / steps * 1e3
        flops = 2.0 * M * H * 2 * F if kind.startswith("fc1") else 2.0 * M * F * H
        out[kind] = {"entry": order[i][0], "us": round(us, 1), "tflops": round(flops / us / 1e6, 1)}
    return out


def router_run(w, steps, warmup):
    """TopKRouter forward + backward (router.py:358-380) at the workload's size."""
    from torchturbo_amd import _lib as L
    from torchturbo_amd import configs as C
    from torchturbo_amd.dispatch import OpPolicy, get_or_create_ops
    from torchturbo_amd.moe import MoEConfig, TopKRouter
    from torchturbo_amd.runtime import CudaRuntime

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    get_or_create_ops(device_runtime=CudaRuntime(), default_policy=OpPolicy.CUSTOM)
    cfg = MoEConfig(
        hidden_size=w.hidden, num_moe_experts=w.experts, moe_router_topk=w.topk,
        moe_router_pre_softmax=w.pre_softmax, moe_router_score_function=w.score_function,
        moe_router_num_groups=w.num_groups, moe_router_group_topk=w.group_topk,
        moe_router_topk_scaling_factor=w.scaling_factor, params_dtype=w.dtype,
        moe_router_enable_expert_bias=w.expert_bias, moe_router_dtype="fp32",
        moe_aux_loss_coeff=1e-3, moe_z_loss_coeff=1e-3, perform_initialization=False,
    )
    router = TopKRouter(cfg).to(dev)
    with torch.no_grad():
        router.weight.normal_(0.0, w.hidden ** -0.5)
    hidden = C.make_hidden(w, device=dev).requires_grad_()
    g = torch.Generator(device=dev).manual_seed(w.seed + 3)
    gp = torch.randn(w.tokens, w.experts, device=dev, generator=g)

    def step():
        router.weight.grad = None
        hidden.grad = None
        probs, _, _, _ = router(hidden)
        (probs * gp).sum().backward()

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    timer = L.KernelTimer(ROUTER_ENTRIES)
    L.set_timer(timer)
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    L.set_timer(None)
    return (t1 - t0) * 1e3 / steps, timer.elapsed_ms(), router._can_fuse_gate(hidden)


def router_line(w, args):
    ms, kernels, fused = router_run(w, args.steps, args.warmup)
    T, H, E = w.tokens, w.hidden, w.experts
    avg = {n: round(v[1] / v[0] * 1e3, 1) for n, v in kernels.items() if v[0]}
    gate_us = avg.get("tt_router_gate_fwd")
    gate = None
    if gate_us:
        flops = 2.0 * T * H * E
        nbytes = T * H * 2 + -(-T // 64) * E * H * 2 + T * E * 9 + T * w.topk * 8
        gate = {"bound": "latency", "kernel": "tt_router_gate_fwd", "avg_launch_us": gate_us,
                "achieved_tflops": round(flops / gate_us / 1e6, 1),
                "achieved_gbs": round(nbytes / gate_us / 1e3, 1)}
    return {
        "metric": "router front end fwd+bwd tokens/sec (gating linear + top-k + aux/z-loss sums)",
        "value": round(T / (ms / 1e3), 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 3),
        "higher_is_better": True, "vs_baseline": None, "data": "synthetic",
        "dtype": "bf16 inputs and router weight, fp32 logits",
        "config": {"workload": w.name, "tokens": T, "hidden": H, "experts": E, "topk": w.topk,
                   "router": w.score_function, "router_dtype": "fp32", "fused_gate": fused,
                   "aux_loss_coeff": 1e-3, "z_loss_coeff": 1e-3},
        "kernels_avg_us": avg, "gate": gate,
    }


def dense_compare(w, reps):
    """fc1 / fc2 of the workload through hipBLASLt (torch.matmul / torch.bmm,
    bf16) beside the grouped kernels, with every expert holding M / E rows,
    the same flops. dense: one product over all M rows (fwd y = x W with one
    expert's weight; weight gradient x^T dy). batched: one product per expert
    (fwd x_e W_e, weight gradient x_e^T dy_e, both operands contiguous), the
    grouped problem with uniform loads, plus the transpose of x that the
    batched weight gradient needs. The launches of a shape alternate,
    back to back, ``reps`` times (a launch's time depends on how long the chip
    has been under load, so blocks of one kind would favour whichever ran
    first); median HIP-event time of each kind. Also for counter runs
    (rocprofv3 tells the kernels apart by name)."""
    import statistics

    from torchturbo_amd import _lib as L

    dev = torch.device("cuda", 0)
    M, H, F, E = w.routed_rows, w.hidden, w.ffn, w.experts
    g = torch.Generator(device=dev).manual_seed(1)
    cnt = torch.full((E,), M // E, dtype=torch.int64, device=dev)
    cnt[0] += M - int(cnt.sum())
    me = M // E
    st = L.stream(dev)
    out = {}
    for name, K, N in (("fc1", H, 2 * F), ("fc2", F, H)):
        x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
        dy = torch.randn(M, N, generator=g, device=dev).to(torch.bfloat16)
        wt = (torch.randn(E, K, N, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        dw = torch.empty_like(wt)
        dwd = torch.empty(K, N, dtype=torch.bfloat16, device=dev)
        runs = {
            "dense_fwd": lambda: torch.matmul(x, wt[0], out=y),
            "dense_wgrad": lambda: torch.matmul(x.t(), dy, out=dwd),
        }
        if me * E == M:
            # hipBLASLt's batched weight gradient takes x_e^T contiguous ([E, K, me]),
            # a layout the layer does not hold: the transpose is timed on its own.
            xt = x.view(E, me, K).transpose(1, 2).contiguous()
            dwb = torch.empty_like(wt)
            runs["batched_fwd"] = lambda: torch.bmm(x.view(E, me, K), wt, out=y.view(E, me, N))
            runs["batched_wgrad"] = lambda: torch.bmm(xt, dy.view(E, me, N), out=dwb)
            runs["transpose_x"] = lambda: xt.copy_(x.view(E, me, K).transpose(1, 2))
        runs["grouped_fwd"] = lambda: L.call("tt_gmm_fwd", L.ptr(x), L.ptr(wt), L.TT_BF16, M, K,
                                             N, E, 0, L.ptr(cnt), L.ptr(y), st)
        runs["grouped_wgrad"] = lambda: L.call("tt_gmm_wgrad", L.ptr(x), L.ptr(dy), L.TT_BF16, M,
                                               K, N, E, 0, L.ptr(cnt), L.ptr(dw), st)
        for fn in runs.values():
            fn()
        torch.cuda.synchronize()
        ev = {kind: [] for kind in runs}
        for _ in range(reps):
            for kind, fn in runs.items():
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                fn()
                b.record()
                ev[kind].append((a, b))
        torch.cuda.synchronize()
        for kind, pairs in ev.items():
            us = statistics.median(a.elapsed_time(b) for a, b in pairs) * 1e3
            out[f"{name}_{kind}"] = {"us": round(us, 1)}
            if kind != "transpose_x":
                out[f"{name}_{kind}"]["tflops"] = round(2.0 * M * K * N / us / 1e6, 1)
        del runs, x, dy, wt, y, dw, dwd
        torch.cuda.empty_cache()
    return {"part": "dense-compare", "workload": w.name, "rows": M, "experts": E,
            "shapes": {"fc1": [M, H, 2 * F], "fc2": [M, F, H]}, "results": out}


def cpu_baseline(w, budget_s):
    """The CPU oracle (the reference's native composition) on a token sample."""
    from dataclasses import replace

    from oracle import layer as o_layer
    from oracle.fp8 import dequantize_experts
    from torchturbo_amd import configs as C

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    full = C.resolve(w)
    w1, w2 = C.make_weights(full)
    if full.fp8:
        q1, s1 = C.fp8_blocks(w1.transpose(1, 2).contiguous())
        q2, s2 = C.fp8_blocks(w2.transpose(1, 2).contiguous())
        fp8 = {"q1": q1, "s1": s1, "q2": q2, "s2": s2,
               "m1": dequantize_experts(q1, s1).requires_grad_(),
               "m2": dequantize_experts(q2, s2).requires_grad_()}
        w1 = w2 = None
    else:
        fp8 = None
        w1.requires_grad_()
        w2.requires_grad_()
    cfg = o_layer.RoutingConfig(topk=w.topk, pre_softmax=w.pre_softmax,
                                score_function=w.score_function, num_groups=w.num_groups,
                                group_topk=w.group_topk, scaling_factor=w.scaling_factor)
    bias = C.make_expert_bias(full)
    tokens = 128
    result = None
    while True:
        sw = replace(full, tokens=tokens, logits="zipf" if full.logits == "varlen" else full.logits)
        hidden = C.make_hidden(sw).requires_grad_()
        logits = C.make_logits(sw).requires_grad_()
        grad = C.make_grad(sw)
        t0 = time.perf_counter()
        out = o_layer.moe_layer(hidden, logits, w1, w2, cfg, expert_bias=bias, fp8=fp8)
        out.backward(grad)
        dt = time.perf_counter() - t0
        result = (tokens, dt)
        if dt * 2.2 > budget_s or tokens * 2 > full.tokens:
            break
        tokens *= 2
    tokens, dt = result
    return {
        "value": round(tokens / dt, 2),
        "unit": "tokens/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"{tokens} of {full.tokens} tokens of the {full.name} layer "
                   f"(all {full.experts} experts, full weights), one fwd+bwd, "
                   f"{dt:.2f} s, torch {torch.__version__} CPU, {cores} threads"),
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU (EP=1); --gpus must be 1",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    from torchturbo_amd import configs as C

    w = C.resolve(C.WORKLOADS[args.workload])
    if args.part == "router":
        print(json.dumps(router_line(w, args)), flush=True)
        return
    if args.part == "dense-compare":
        print(json.dumps(dense_compare(w, max(args.steps, 1))), flush=True)
        return
    ms, kernels, order = gpu_run(w, args.steps, args.warmup)
    tokens_per_s = w.tokens / (ms / 1e3)

    gemm_launches = sum(kernels.get(n, (0, 0.0))[0] for n in GEMM_ENTRIES)
    gemm_ms = sum(kernels.get(n, (0, 0.0))[1] for n in GEMM_ENTRIES)
    flops_step = w.gemm_flops_fwd_bwd()
    per_launch_flops = flops_step * args.steps / max(gemm_launches, 1)
    avg_launch_s = gemm_ms / 1e3 / max(gemm_launches, 1)
    achieved_tflops = per_launch_flops / avg_launch_s / 1e12 if avg_launch_s > 0 else 0.0

    perm_n, perm_ms = kernels.get("tt_permute_scatter", (0, 0.0))
    unperm_n, unperm_ms = kernels.get("tt_unpermute_gather", (0, 0.0))
    pass_bytes = w.permute_bytes()
    perm_gbs = pass_bytes / (perm_ms / 1e3 / perm_n) / 1e9 if perm_n else None
    unperm_gbs = pass_bytes / (unperm_ms / 1e3 / unperm_n) / 1e9 if unperm_n else None
    # SwiGLU x probs: fwd reads [M, 2F] and the fp32 probs, writes [M, F]; bwd
    # reads [M, 2F], [M, F] and the probs, writes [M, 2F] and fp32 d-probs.
    M, F2, b = w.routed_rows, 2 * w.ffn, 2
    sw_bytes = {"tt_swiglu_fwd": M * F2 * b + M * 4 + M * w.ffn * b,
                "tt_swiglu_bwd": 2 * M * F2 * b + M * w.ffn * b + 8 * M}
    sw_gbs = {}
    for name, nbytes in sw_bytes.items():
        n, t_ms = kernels.get(name, (0, 0.0))
        sw_gbs[name] = round(nbytes / (t_ms / 1e3 / n) / 1e9, 1) if n else None

    line = {
        "metric": "MoE layer fwd+bwd tokens/sec on 1 MI355X; grouped-GEMM % MFMA peak",
        "value": round(tokens_per_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8-e4m3 weights, bf16" if w.fp8 else str(w.dtype).replace("torch.", "").replace("bfloat16", "bf16"),
        "data": "synthetic",
        "config": {
            "workload": w.name, "tokens": w.tokens, "hidden": w.hidden, "experts": w.experts,
            "topk": w.topk, "ffn": w.ffn, "router": w.score_function,
            "routed_rows": w.routed_rows, "gemm_tflop_per_step": round(flops_step / 1e12, 4),
            "parallelism": "ep1",
        },
        "roofline": {
            "bound": "mfma",
            "kernel": "grouped GEMM (tt_gmm_*, row-gathering ones included; fc1/fc2 fwd, "
                      "dgrad, wgrad)",
            "achieved": round(achieved_tflops, 1),
            "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved_tflops / MFMA_BF16_PEAK_TFLOPS, 4),
            "traffic": measured_traffic(w.name),
            "traffic_unit": "bytes/launch",
            "launches": gemm_launches,
            "avg_launch_us": round(avg_launch_s * 1e6, 1),
            "gemm_ms_per_step": round(gemm_ms / args.steps, 3),
            "per_gemm": per_gemm(w, order, args.steps),
        },
        "permute": {
            "bound": "hbm", "unit": "GB/s", "peak": HBM_PEAK_GBS,
            "permute_scatter_gbs": None if perm_gbs is None else round(perm_gbs, 1),
            "permute_scatter_calls_per_step": perm_n / args.steps,
            "unpermute_gather_gbs": None if unperm_gbs is None else round(unperm_gbs, 1),
            "bytes_per_pass": pass_bytes,
            "swiglu_fwd_gbs": sw_gbs["tt_swiglu_fwd"],
            "swiglu_bwd_gbs": sw_gbs["tt_swiglu_bwd"],
            "swiglu_bytes": sw_bytes,
        },
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(w, args.cpu_budget_s)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
