"""Write the golden fixtures of this directory (run from the repo root).

* ``routing_cases.json`` — tiny routing inputs with their packed-row maps
  computed by brute-force enumeration of (expert, token) pairs
  (``oracle/route_np.py::brute_force``) and their top-k ids for fp32 logits.
* ``router_loss_cases.json`` — tiny fp32 logits with padding rows and the
  aux-loss / z-loss sums (per-expert score sums, top-k counts, sum of squared
  log-sum-exps) by per-row brute force in Python floats.
* ``toy_layer.npz`` — configuration 0 of the benchmark definition (512
  tokens, hidden 256, 8 experts, top-2, ffn 512, fp32, logits N(0, 1), weights
  N(0, 0.02), seed 0): the CPU oracle layer's routing ids, per-expert counts,
  and the first 64 tokens of the output and of the hidden-state gradient,
  plus whole-tensor norms of the output and every gradient.

The reference package itself cannot be imported here (it needs Python 3.11),
so these vectors come from the oracle's restatement; they pin the oracle
against regressions and give the GPU tests fixed expected values.
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import layer as o_layer  # noqa: E402
from oracle import route_np  # noqa: E402
from oracle.native_providers import routing as o_route  # noqa: E402
from torchturbo_amd import configs as C  # noqa: E402


def routing_cases():
    cases = []
    rng = np.random.default_rng(1234)
    for T, E, k in ((1, 2, 1), (5, 4, 2), (9, 8, 3), (16, 8, 8), (12, 16, 4), (7, 32, 6)):
        logits = rng.standard_normal((T, E)).astype(np.float32)
        ids = o_route.topk_softmax_with_capacity(torch.from_numpy(logits), k)[2].numpy()
        rows, token_of_row, counts, offsets = route_np.brute_force(ids, E)
        cases.append({
            "T": T, "E": E, "k": k, "logits": logits.tolist(), "ids": ids.tolist(),
            "row_indices": rows.tolist(), "token_of_row": token_of_row.tolist(),
            "counts": counts.tolist(),
        })
    with open(os.path.join(HERE, "routing_cases.json"), "w") as f:
        json.dump(cases, f)


def _loss_sums_brute_force(logits, k, score_function, pad):
    """Per-row loops in Python floats: scores by definition, the top-k set by a
    full sort (larger first, lower id on equal scores), log-sum-exp with math."""
    import math
    T, E = len(logits), len(logits[0])
    psum, cnt, z = [0.0] * E, [0] * E, 0.0
    for t in range(T):
        if pad[t]:
            continue
        row = logits[t]
        m = max(row)
        if score_function == "softmax":
            ex = [math.exp(v - m) for v in row]
            sc = [v / sum(ex) for v in ex]
        else:
            f = ((lambda v: 1.0 / (1.0 + math.exp(-v))) if score_function == "sigmoid"
                 else (lambda v: math.sqrt(v if v > 20.0 else math.log1p(math.exp(v)))))
            r = [f(v) for v in row]
            sc = [v / (sum(r) + 1e-20) for v in r]
        for e in range(E):
            psum[e] += sc[e]
        for e in sorted(range(E), key=lambda e: (-sc[e], e))[:k]:
            cnt[e] += 1
        z += (m + math.log(sum(math.exp(v - m) for v in row))) ** 2
    return psum, cnt, z


def router_loss_cases():
    """Aux-loss / z-loss sums (models/modules/moe/moe_utils.py:15-70) of tiny fp32
    logits with padding rows, by brute force."""
    cases = []
    rng = np.random.default_rng(4321)
    for T, E, k, sf in ((6, 4, 2, "softmax"), (9, 8, 3, "sigmoid"), (7, 16, 4, "sqrtsoftplus"),
                        (12, 32, 8, "softmax"), (5, 64, 6, "sigmoid")):
        logits = (rng.standard_normal((T, E)) * 2).astype(np.float32)
        pad = (rng.random(T) < 0.25).tolist()
        psum, cnt, z = _loss_sums_brute_force(logits.astype(np.float64).tolist(), k, sf, pad)
        cases.append({"T": T, "E": E, "k": k, "score_function": sf, "logits": logits.tolist(),
                      "padding_mask": pad, "prob_sum": psum, "tokens_per_expert": cnt,
                      "z_sum": z})
    with open(os.path.join(HERE, "router_loss_cases.json"), "w") as f:
        json.dump(cases, f)


def toy_layer():
    w = C.TOY
    hidden, logits = C.make_hidden(w), C.make_logits(w)
    w1, w2 = C.make_weights(w)
    grad = C.make_grad(w)
    h = hidden.clone().requires_grad_()
    lg = logits.clone().requires_grad_()
    a = w1.clone().requires_grad_()
    b = w2.clone().requires_grad_()
    out, trace = o_layer.moe_layer(h, lg, a, b, o_layer.RoutingConfig(topk=w.topk), trace=True)
    out.backward(grad)
    np.savez_compressed(
        os.path.join(HERE, "toy_layer.npz"),
        ids=trace.expert_indices.numpy().astype(np.int64),
        counts=trace.tokens_per_expert.numpy().astype(np.int64),
        out_head=out.detach()[:64].numpy(),
        dhidden_head=h.grad[:64].numpy(),
        norms=np.array([out.detach().norm().item(), h.grad.norm().item(), lg.grad.norm().item(),
                        a.grad.norm().item(), b.grad.norm().item()], dtype=np.float64),
    )


if __name__ == "__main__":
    routing_cases()
    router_loss_cases()
    toy_layer()
    print("fixtures written to", HERE)
