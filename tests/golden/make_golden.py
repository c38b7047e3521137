"""Writes the golden fixtures of this directory.

Run from the repository root:  python tests/golden/make_golden.py

* known_answers.json -- inputs and expected outputs transcribed from the
  reference's own unit-test assertions (file:line in each entry).
* adam_libtorch_cases.json -- the reference's LibTorch Adam validation cases
  (libtorch-validation/src/validation/optimizers/adam.rs), with the expected
  parameters recomputed by torch.optim.Adam in float64 on the CPU: the
  reference compares against LibTorch 2.0.0 CPU, which is not available here,
  and torch's Adam is the same library's algorithm.  Tolerance of those tests:
  |ours - torch| <= 1e-4 * |torch| or <= 1e-4 (validation/core.rs:138-141).
* ltv_patterns.json -- the input patterns of the LibTorch forward/gradient
  validations for relu / add / div, with torch float32 CPU outputs.

The generator needs torch (CPU) only; the fixtures are data and are read by
tests/ without torch.
"""
from __future__ import annotations

import json
import pathlib

import torch

HERE = pathlib.Path(__file__).resolve().parent


def known_answers() -> dict:
    return {
        "matmul_2x2": {
            "source": "train-station/src/tensor/ops/matmul/mod.rs:1145-1195",
            "a": [1.0, 2.0, 3.0, 4.0], "b": [5.0, 6.0, 7.0, 8.0], "shape": [2, 2],
            "out": [19.0, 22.0, 43.0, 50.0], "grad_output": [1.0, 1.0, 1.0, 1.0],
            "grad_a": [11.0, 15.0, 11.0, 15.0], "grad_b": [4.0, 4.0, 6.0, 6.0],
        },
        "linear_bias_grad": {
            "source": "train-station/src/tensor/ops/add.rs:893-946",
            "input": [1.0, 2.0, 3.0, 4.0, 5.0, 6.0], "input_shape": [2, 3],
            "weight": [i * 0.1 for i in range(1, 13)], "weight_shape": [3, 4],
            "bias": [0.1, 0.2, 0.3, 0.4], "bias_grad": [2.0, 2.0, 2.0, 2.0], "tol": 1e-6,
        },
        "sum_forward": {
            "source": "train-station/src/tensor/reductions/sum.rs:313-327",
            "x": [i * 0.5 for i in range(6)], "shape": [2, 3], "sum": 7.5, "tol": 1e-6,
        },
        "sum_all_ones_grad": {
            "source": "train-station/src/tensor/reductions/sum.rs:328-345",
            "x": [0.0, 1.0, 2.0, 3.0], "shape": [2, 2], "grad": [1.0, 1.0, 1.0, 1.0],
        },
        "sum_chain_grad": {
            "source": "train-station/src/tensor/reductions/sum.rs:346-362",
            "x": [1.0, 2.0, 3.0, 4.0], "shape": [2, 2], "mul": 2.0, "add": 1.0,
            "grad": [2.0, 2.0, 2.0, 2.0],
        },
        "sum_21": {
            "source": "train-station/src/tensor/reductions/sum.rs:363-380",
            "x": [1.0, 2.0, 3.0, 4.0, 5.0, 6.0], "shape": [2, 3], "sum": 21.0,
        },
        "sum_276": {
            "source": "train-station/src/tensor/reductions/sum.rs:404-420",
            "x": [float(i) for i in range(24)], "shape": [2, 3, 4], "sum": 276.0,
        },
        "mean_forward": {
            "source": "train-station/src/tensor/reductions/mean.rs:237-251",
            "x": [float(i) for i in range(6)], "shape": [2, 3], "mean": 2.5, "tol": 1e-6,
        },
        "mean_grad": {
            "source": "train-station/src/tensor/reductions/mean.rs:252-266",
            "x": [1.0, 3.0, 5.0, 7.0], "shape": [4], "grad": [0.25, 0.25, 0.25, 0.25],
        },
        "mean_3_5": {
            "source": "train-station/src/tensor/reductions/mean.rs:267-284",
            "x": [1.0, 2.0, 3.0, 4.0, 5.0, 6.0], "shape": [2, 3], "mean": 3.5, "tol": 1e-6,
        },
        "relu_forward": {
            "source": "train-station/src/tensor/ops/relu.rs:280-291",
            "x": [-1.0, 0.0, 2.5], "out": [0.0, 0.0, 2.5],
        },
        "pow_scalar_forward": {
            "source": "train-station/src/tensor/ops/pow.rs:546-558",
            "x": [1.0, 2.0, 3.0, 4.0], "exponent": 2.0, "out": [1.0, 4.0, 9.0, 16.0],
        },
    }


def _adam_run(p0, steps, loss, **cfg) -> list[list[float]]:
    p = torch.tensor(p0, dtype=torch.float64, requires_grad=True)
    opt = torch.optim.Adam([p], lr=cfg.get("lr", 1e-3), betas=(cfg.get("beta1", 0.9), cfg.get("beta2", 0.999)),
                           eps=cfg.get("eps", 1e-8), weight_decay=cfg.get("weight_decay", 0.0),
                           amsgrad=cfg.get("amsgrad", False))
    traj = []
    for _ in range(steps):
        opt.zero_grad()
        loss(p).backward()
        opt.step()
        traj.append(p.detach().tolist())
    return traj


def adam_cases() -> dict:
    lin = lambda p: (p * 2.0 + 1.0).sum()  # noqa: E731  adam.rs:143-147
    quad = lambda p: ((p - 0.5) * (p - 0.5)).sum()  # noqa: E731  adam.rs:1108-1116
    src = "libtorch-validation/src/validation/optimizers/adam.rs"
    cases = {}
    n12 = [i * 0.01 - 0.5 for i in range(12)]
    cases["single_parameter"] = {"source": f"{src}:65-160,1280-1286", "shape": [3, 4], "p0": n12,
                                 "loss": "sum(2p+1)", "config": {}, "steps": 3}
    cases["weight_decay"] = {"source": f"{src}:1333-1342", "shape": [3, 4], "p0": n12,
                             "loss": "sum(2p+1)", "config": {"weight_decay": 0.01}, "steps": 3}
    n9 = [i * 0.01 - 0.5 for i in range(9)]
    cases["amsgrad"] = {"source": f"{src}:1740-1770", "shape": [3, 3], "p0": n9, "loss": "sum(2p+1)",
                        "config": {"amsgrad": True}, "steps": 10}
    cases["regular_10"] = {"source": f"{src}:1740-1770", "shape": [3, 3], "p0": n9, "loss": "sum(2p+1)",
                           "config": {}, "steps": 10}
    for shape in ([3], [2, 2]):
        n = 1
        for d in shape:
            n *= d
        cases[f"long_term_{'x'.join(map(str, shape))}"] = {
            "source": f"{src}:1058-1157,1629-1641", "shape": shape, "p0": [i * 0.1 for i in range(n)],
            "loss": "sum((p-0.5)*(p-0.5))", "config": {}, "steps": 50}
    for c in cases.values():
        fn = lin if c["loss"] == "sum(2p+1)" else quad
        p0 = [float(torch.tensor(v, dtype=torch.float32)) for v in c["p0"]]  # f32 inputs as the reference
        c["p0"] = p0
        c["torch_trajectory"] = _adam_run(p0, c["steps"], fn, **c["config"])
        c["rtol"] = 1e-4
        c["atol"] = 1e-4
    return cases


def ltv_patterns() -> dict:
    src = "libtorch-validation/src/validation/tensor/ops"
    n = 24
    relu_x = torch.arange(n, dtype=torch.float32) * torch.tensor(0.2, dtype=torch.float32) - 1.0
    a = torch.arange(n, dtype=torch.float32) * torch.tensor(0.1, dtype=torch.float32)
    d_a = a + 2.0
    d_b = torch.arange(n, dtype=torch.float32) * torch.tensor(0.2, dtype=torch.float32) + 1.0
    return {
        "relu": {"source": f"{src}/relu.rs:6-70", "x": relu_x.tolist(),
                 "out": torch.relu(relu_x).tolist(),
                 "grad_of_sum": (relu_x > 0).to(torch.float32).tolist()},
        "add": {"source": f"{src}/add.rs:231-340", "a": a.tolist(), "b": a.tolist(),
                "out": (a + a).tolist()},
        "div": {"source": f"{src}/div.rs:132-180", "a": d_a.tolist(), "b": d_b.tolist(),
                "out": (d_a / d_b).tolist()},
    }


def main() -> None:
    (HERE / "known_answers.json").write_text(json.dumps(known_answers(), indent=1))
    (HERE / "adam_libtorch_cases.json").write_text(json.dumps(adam_cases(), indent=1))
    (HERE / "ltv_patterns.json").write_text(json.dumps(ltv_patterns(), indent=1))
    print("wrote", sorted(p.name for p in HERE.glob("*.json")))


if __name__ == "__main__":
    main()
